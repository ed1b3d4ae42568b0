// Attention: flash-attention prefill and split-K KV-cache decode.
//
// Reference: mat_head_gen_t::forward (mat_mha_t.hpp:45-74) materialises the full
// S = Q'K / sqrt(d) matrix, masks j > i to -inf (:58-67), runs hsoftmax and multiplies
// V P'.  Decoding (test_transformer_t::predict, transformer_test.hpp:194-242) recomputes
// the whole prefix every step.  Here:
//  * prefill never materialises S: each workgroup owns 64 queries (16 per wave), streams
//    64-key K/V tiles through LDS and keeps an online softmax.  The wave computes
//    S^T = K Q^T on the matrix cores so that the probabilities land in exactly the operand
//    layout of the second product (O += P V, or O^T += V^T P^T for bf16) -- P never leaves
//    registers.
//  * decode splits each (sequence, head)'s keys over workgroups (flash-decoding), each
//    reading its K/V slice once from HBM, then merges the partial softmaxes by log-sum-exp.
#include "jas_common.hpp"

#include <cfloat>
#include <atomic>
#include <mutex>
#include <type_traits>
#include <unordered_map>

namespace jas {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c)
{
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
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
    // key split (non-causal only): work item `split` attends over keys
    // [split * kchunk, min(Sk, (split + 1) * kchunk)) and writes its unnormalised output with
    // its row max and row sum to part[split][b*H + h][q][D + 2]; a merge kernel combines them
    int nsplit = 1, kchunk = 0;
    float *part = nullptr;
    // > 0: the CU count of a launch whose workgroups sit two to a CU (see fa_work_item)
    int fold = 0;
};

// waves per workgroup (16 queries each), measured with the heaviest-first work order: 4 or
// 16 waves are slower for bf16, and 8 beats 4 for fp32 (by 17 % at D = 128)
constexpr int FA_WAVES = 8;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));


// 2^x on the hardware exp unit (v_exp_f32): results below 2^-126 flush to zero.  Used for
// softmax terms 2^(s - max) <= 1, where such terms cannot change a sum that contains 1.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
// max over the four 16-lane rows of a wave (lanes l, l^16, l^32, l^48): gfx950's
// permlane swaps exchange rows in registers (no LDS round trip, unlike a shuffle)
__device__ __forceinline__ float max_across_rows(float v)
{
    const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float m = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane16_swap(__float_as_uint(m), __float_as_uint(m), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// a 16-byte chunk as a native vector (HIP's uint4 struct defeats register promotion)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Work item of this workgroup: query blocks in order of decreasing causal cost (the last
// query block first), then (batch, head).  Workgroups are dispatched in id order, so the
// heaviest items start first and the light ones fill the slots that free up -- the longest
// chain is about one heavy item (interleaving heavy and light items per head left heavy
// ones starting late: about 1.4x longer for the causal config-3 shape).  Consecutive ids go
// round robin to the 8 XCDs, so with B*H a multiple of 8 the query blocks of one head,
// which share its K/V, stay on one XCD's L2.
// fold = C (the CU count, when workgroups sit two to a CU): ids i and i + C start together
// on one CU, so ranks [C, 2C) are taken in reverse groups of 8 (the XCD of each rank kept):
// the heaviest first-round items share their CU with the lightest of the second 256 rather
// than with the next heaviest (a workgroup timeline of the config-3 launch showed CUs paired
// 16 + 12 key tiles against others at 12 + 6).
__device__ __forceinline__ bool fa_work_item(int nqb, int BH, int nsplit, int fold, int &bh, int &qb, int &split)
{
    const int id = (int)blockIdx.x;
    if (id >= nqb * BH * nsplit) return false;
    split = id / (nqb * BH);
    int rem = id % (nqb * BH);
    if (fold > 0 && rem >= fold && rem < 2 * fold) rem = fold + (fold / 8 - 1 - (rem - fold) / 8) * 8 + (rem & 7);
    qb = nqb - 1 - rem / BH;
    bh = rem % BH;
    return true;
}

// One workgroup = 64 queries of one (batch, head), 16 per wave.  Key/value tiles of 64
// rows are double-staged: the global loads of tile t+1 are issued into registers before
// tile t is computed from LDS, so HBM latency hides behind the matrix work.  Rows past
// Sk are read clamped (finite data) and masked to probability 0.  fp32: S^T = K Q^T and
// O += P V on v_mfma_f32_16x16x4_f32.  bf16: S^T = K Q^T and O^T += V^T P^T on
// v_mfma_f32_16x16x32_bf16 (fp32 accumulate, softmax in fp32, P rounded to bf16 for the
// second product), so every accumulator entry of a lane belongs to the lane's own query and
// the rescale needs no cross-lane traffic; the reduction index of each product is permuted
// identically in both operands so that S lands in the P operand's registers with no shuffle.
template <int D, bool BF16, int BK, int NW = FA_WAVES>
__global__ void __launch_bounds__(64 * NW, (NW == 8 && D <= 64) ? 4 : 1) flash_prefill_kernel(const PrefillArgs p)
{
    constexpr int FA_NW = NW, FA_BQ = 16 * FA_NW;
    constexpr int NT = 64 * FA_NW;
    using T = typename std::conditional<BF16, uint16_t, float>::type;
    constexpr int EPC = 16 / (int)sizeof(T);    // elements per 16-byte chunk
    constexpr int KLD = D + (BF16 ? 8 : 4);    // padded row strides (elements)
    // bf16 V rows are read with the transposing ds_read_b64_tr_b16: 16 rows x 4 column chunks
    // per 16 lanes; a 40-dword row stride puts the four rows of a lane quad on disjoint banks
    constexpr int KLDV = BF16 ? D + 16 : KLD;
    constexpr int CPR = D / EPC;                // 16-byte chunks per key row
    constexpr int NCH = BK * CPR;            // 16-byte chunks per tile and tensor
    constexpr int NLD = (NCH + NT - 1) / NT;    // chunks per thread per tensor and tile
    constexpr int NC = D / 16;                  // 16-row blocks of the head dim (output)
    constexpr int NJ = BK / 16;                 // 16-key blocks of a tile
    static_assert(NCH % NT == 0 || NLD == 1, "tile/thread mismatch");
    // two tile buffers: tile t+1 is written while tile t is read, one barrier per tile
    __shared__ __attribute__((aligned(16))) T Ks[2][BK * KLD];
    // V row-major [BK][D] like K: the O = P V product reads its operand per key row (fp32:
    // one float per lane and key; bf16: the LDS transpose read, ds_read_b64_tr_b16)
    __shared__ __attribute__((aligned(16))) T Vt[2][BK * KLDV];

    const int tid = threadIdx.x, lane = tid & 63, r16 = lane & 15, g = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar branches
    int bh, qb, split;
    const int nqb = (p.Sq + FA_BQ - 1) / FA_BQ;
    if (!fa_work_item(nqb, p.B * p.H, p.nsplit, p.fold, bh, qb, split)) return;
    const int b = bh / p.H, h = bh % p.H;
    const int q0 = qb * FA_BQ + w * 16;
    const int qi = q0 + r16;  // this lane's query (column of S^T)
    const int shift = p.Sk - p.Sq;
    const int qq = qi < p.Sq ? qi : p.Sq - 1;
    const long qbase = (long)b * p.q_sb + (long)h * p.q_sh + (long)qq * p.q_ss;

    const int q_last = min(qb * FA_BQ + FA_BQ - 1, p.Sq - 1);
    // keys of this work item: [k_lo, k_end)
    const int k_lo = p.nsplit > 1 ? split * p.kchunk : 0;
    const int k_end = p.nsplit > 1 ? min(p.Sk, k_lo + p.kchunk) : p.causal ? min(p.Sk, q_last + shift + 1) : p.Sk;
    // keys this wave can see at all (causal): [0, wave_kend)
    const int wave_kend = min(k_end, p.causal ? min(p.Sk, min(q0 + 15, p.Sq - 1) + shift + 1) : p.Sk);
    const long kbase = (long)b * p.k_sb + (long)h * p.k_sh;

    // staging: chunk `it` of this thread is (key row, 16-byte column) of the 64-row tile
    // two register sets: tile t+1 is in one while tile t+2 is in flight in the other
    u32x4 kra[NLD], vra[NLD], krb[NLD], vrb[NLD];
    long goff[NLD];
#pragma unroll
    for (int it = 0; it < NLD; ++it) {
        const int idx = min(tid + it * NT, NCH - 1);
        goff[it] = kbase + (long)(idx / CPR) * p.k_ss + (idx % CPR) * EPC;
    }
    // rows past Sk are read clamped to the last row (finite data, masked below)
#define FA_GLOAD(KV0, KR, VR)                                                                \
    if ((KV0) + BK <= p.Sk) {                                                           \
        const long o0 = (long)(KV0) * p.k_ss;                                              \
        _Pragma("unroll") for (int it = 0; it < NLD; ++it)                                 \
        {                                                                                  \
            KR[it] = *(const u32x4 *)((const T *)p.K + goff[it] + o0);                     \
            VR[it] = *(const u32x4 *)((const T *)p.V + goff[it] + o0);                     \
        }                                                                                  \
    } else {                                                                               \
        _Pragma("unroll") for (int it = 0; it < NLD; ++it)                                 \
        {                                                                                  \
            const int idx = min(tid + it * NT, NCH - 1), key = idx / CPR, ch = idx % CPR; \
            const long off = kbase + (long)min((KV0) + key, p.Sk - 1) * p.k_ss + ch * EPC; \
            KR[it] = *(const u32x4 *)((const T *)p.K + off);                               \
            VR[it] = *(const u32x4 *)((const T *)p.V + off);                               \
        }                                                                                  \
    }

    floatx4 oacc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) oacc[c] = floatx4{0.f, 0.f, 0.f, 0.f};
    // running max (raw score units) and this lane's partial row sum: the lanes g = 0..3 of
    // one query each sum their own keys; the four partials are combined once at the end
    float m_run = -INFINITY, l_part = 0.f;
    // bf16: the row sums come out of the matrix core too (P times a ones operand), already in
    // the accumulator's query layout -- no per-score adds, no final shuffles
    floatx4 lacc = floatx4{0.f, 0.f, 0.f, 0.f};
    const float sl2 = p.scale_log2;
    // bf16: the exponent base mb of this lane's query (exponent units, shared by the row's
    // four lanes) and this lane's running max of its scores relative to it
    float mb = 0.f, m_lane = -INFINITY;

    // Q fragments (B operand of S^T = K Q^T), raw (the scale is applied in the exponent)
    float4 qf[BF16 ? 1 : NC];
    bf16x8 qb16[BF16 ? D / 32 : 1];
    if constexpr (BF16) {
#pragma unroll
        for (int c = 0; c < D / 32; ++c)
            qb16[c] = *(const bf16x8 *)((const uint16_t *)p.Q + qbase + 32 * c + 8 * g);
    } else {
#pragma unroll
        for (int c = 0; c < NC; ++c) qf[c] = *(const float4 *)((const float *)p.Q + qbase + 16 * c + 4 * g);
    }

#define FA_LSTORE(BUF, KR, VR)                                                               \
    _Pragma("unroll") for (int it = 0; it < NLD; ++it)                                     \
    {                                                                                      \
        const int idx = tid + it * NT, key = idx / CPR, ch = idx % CPR;                    \
        if (NCH % NT != 0 && idx >= NCH) break;                                            \
        *(u32x4 *)(&Ks[BUF][key * KLD + ch * EPC]) = KR[it];                               \
        if constexpr (BF16) {                                                                   \
            *(u32x4 *)(&Vt[BUF][key * KLDV + ch * EPC]) = VR[it];                              \
        } else { /* fp32 V rows interleaved: element d at (d % 16) * NC + d / 16 */            \
            _Pragma("unroll") for (int e = 0; e < 4; ++e)                                      \
            {                                                                                  \
                const int d = ch * EPC + e;                                                    \
                Vt[BUF][key * KLDV + (d % 16) * NC + d / 16] = __uint_as_float(VR[it][e]);    \
            }                                                                                  \
        }                                                                                      \
    }

    // Pipeline: tile t is computed from LDS buffer t%2 while tile t+1 waits in registers
    // (staged into the other buffer at the top of step t) and tile t+2 is in flight from HBM
    // into the other register set -- loads are issued two tiles ahead of their use.
    // Register set A holds the odd tiles, B the even ones (after tile 0).
    // Every step issues the same loads whether or not its tile exists (a tile past the work
    // item's last one re-reads the last, an L2 hit): with a path-independent number of loads in
    // flight the compiler's wait counts only cover the tile being staged, and the loads of the
    // next two tiles stay in flight behind the matrix work.  Every work item has keys
    // (k_end > k_lo).
    const int k_last = k_lo + (k_end - k_lo - 1) / BK * BK;
    FA_GLOAD(k_lo, kra, vra)
    FA_LSTORE(0, kra, vra)
    FA_GLOAD(min(k_lo + BK, k_last), kra, vra)
    FA_GLOAD(min(k_lo + 2 * BK, k_last), krb, vrb)
    __syncthreads();
    auto tile = [&](const int kv0, const int buf) __attribute__((always_inline)) {
        const T *Kc = Ks[buf], *Vc = Vt[buf];

        // S^T tile: lane holds S^T[key = kv0 + 16j + 4g + r][query = qi] (raw scores)
        floatx4 s[NJ];
        // bf16: the K fragments of the tile are requested first; the V fragments after the
        // score products have been issued (reusing the K fragments' registers), and their
        // reads complete behind the softmax
        bf16x8 kfr[BF16 ? NJ : 1][BF16 ? D / 32 : 1];
        if constexpr (BF16) {
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int c = 0; c < D / 32; ++c)
                    kfr[j][c] = *(const bf16x8 *)(Kc + (16 * j + r16) * KLD + 32 * c + 8 * g);
        }
        // masking only on tiles that reach past Sk or cross this wave's causal diagonal: key
        // kv0 + 16j + 4g + r is visible iff 16j + r <= lim, one compare per score
        const bool need_mask = kv0 + BK > p.Sk || (p.causal && kv0 + BK - 1 > q0 + shift);
        const int lim = (p.causal ? min(qi + shift, p.Sk - 1) : p.Sk - 1) - kv0 - 4 * g;
        if constexpr (BF16) {
            // raw scores; the NJ key blocks are independent accumulators, innermost so that
            // consecutive matrix ops never wait on each other's result
#pragma unroll
            for (int c = 0; c < D / 32; ++c)
#pragma unroll
                for (int j = 0; j < NJ; ++j)
                    s[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kfr[j][c], qb16[c], c == 0 ? floatx4{0.f, 0.f, 0.f, 0.f} : s[j], 0, 0, 0);
            bf16x8 vfr[NC][NJ / 2];
            // A operand of O^T = V^T P^T for key block m, head-dim block c: lane (n = l%16, g) needs
            // V[key][16c + n] for keys 32m + 4g + 0..3 and 32m + 16 + 4g + 0..3.  The transpose
            // read hands lane n of each 16-lane group element n%4 of the 4-element chunks that
            // lanes n/4 + 4e address (e = 0..3), so lane i addresses row (key base + i/4),
            // columns 16c + 4(i%4) .. +3.
            typedef short s16x4 __attribute__((ext_vector_type(4)));
            typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int m = 0; m < NJ / 2; ++m) {
                    const uint16_t *v0 = Vc + (32 * m + 4 * g + (r16 >> 2)) * KLDV + 16 * c + 4 * (r16 & 3);
                    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)v0);
                    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4 *)(v0 + 16 * KLDV));
                    vfr[c][m] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                }
            if (need_mask) {
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[j][r] = 16 * j + r <= lim ? s[j][r] : -INFINITY;
            }
            // exponent units relative to the base: s <- sl2 s - mb (p = 2^s below)
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) s[j][r] = __builtin_fmaf(s[j][r], sl2, -mb);
            // Lazy rescaling with a per-lane test: the base mb moves only when the row's running
            // max leaves [mb - 64, mb + 8].  Meanwhile p stays below 2^8, numerator and row sum
            // share the base, and O / l is unchanged.  Each lane tests only its own running max
            // (taken after the fma: arithmetic results need no NaN canonicalisation before a
            // max); the row max across the four lanes, and the move itself, are computed only
            // when some lane trips, which for most inputs happens on no tile at all.  A query
            // with no visible key keeps -inf maxima.
            const float m_prev = m_lane;
#pragma unroll
            for (int j = 0; j < NJ; ++j) m_lane = fmaxf(fmaxf(m_lane, fmaxf(s[j][0], s[j][1])), fmaxf(s[j][2], s[j][3]));
            if (__builtin_amdgcn_ballot_w64(m_lane > 8.f || (m_lane < -64.f && m_lane != -INFINITY))) {
                const float row_prev = max_across_rows(m_prev), row = max_across_rows(m_lane);
                if (row > 8.f || (row < -64.f && row != -INFINITY)) {
                    // nothing accumulated yet (row_prev = -inf): factor 0, not 2^-row, which
                    // overflows when the base moves far down
                    const float corr = row_prev == -INFINITY ? 0.f : exp2_fast(-row);
                    mb += row;
                    m_lane -= row;
#pragma unroll
                    for (int j = 0; j < NJ; ++j) s[j] -= row;
#pragma unroll
                    for (int c = 0; c < NC; ++c) oacc[c] *= corr;  // O^T: the lane's own query
                    lacc *= corr;
                }
            }
            // P^T operand for key block m (32 keys): slot t <-> key 32m + 16(t/4) + 4g + t%4,
            // which are exactly s[2m][t] and s[2m+1][t-4] of this lane
            bf16x8 pb[NJ / 2];
#pragma unroll
            for (int m = 0; m < NJ / 2; ++m)
            {
                float e[8];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    e[r] = exp2_fast(s[2 * m][r]);
                    e[4 + r] = exp2_fast(s[2 * m + 1][r]);
                }
                pb[m] = bf16x8{(__bf16)e[0], (__bf16)e[1], (__bf16)e[2], (__bf16)e[3],
                               (__bf16)e[4], (__bf16)e[5], (__bf16)e[6], (__bf16)e[7]};
            }
            // O^T += V^T P^T; row sums as P^T times a ones operand
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int m = 0; m < NJ / 2; ++m)
                    oacc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vfr[c][m], pb[m], oacc[c], 0, 0, 0);
            const bf16x8 ones = bf16x8{(__bf16)1.f, (__bf16)1.f, (__bf16)1.f, (__bf16)1.f,
                                       (__bf16)1.f, (__bf16)1.f, (__bf16)1.f, (__bf16)1.f};
#pragma unroll
            for (int m = 0; m < NJ / 2; ++m) lacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pb[m], lacc, 0, 0, 0);
        } else {
            // raw scores; the NJ key blocks are independent accumulators (j innermost)
#pragma unroll
            for (int j = 0; j < NJ; ++j) s[j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                float4 kf[NJ];
#pragma unroll
                for (int j = 0; j < NJ; ++j) kf[j] = *(const float4 *)(Kc + (16 * j + r16) * KLD + 16 * c + 4 * g);
#pragma unroll
                for (int j = 0; j < NJ; ++j) s[j] = mfma4(kf[j].x, qf[c].x, s[j]);
#pragma unroll
                for (int j = 0; j < NJ; ++j) s[j] = mfma4(kf[j].y, qf[c].y, s[j]);
#pragma unroll
                for (int j = 0; j < NJ; ++j) s[j] = mfma4(kf[j].z, qf[c].z, s[j]);
#pragma unroll
                for (int j = 0; j < NJ; ++j) s[j] = mfma4(kf[j].w, qf[c].w, s[j]);
            }
            if (need_mask) {
#pragma unroll
                for (int j = 0; j < NJ; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[j][r] = 16 * j + r <= lim ? s[j][r] : -INFINITY;
            }
            float tmax = s[0][0];
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int r = (j == 0 ? 1 : 0); r < 4; ++r) tmax = fmaxf(tmax, s[j][r]);
            tmax = max_across_rows(tmax);
            // lazy rescaling: the base m_run moves only when some query's max has grown by
            // more than 2^8 in exponent units (or was -inf); p = 2^(sl2 (s - m_run)) stays below
            // 256 meanwhile, and numerator and row sum share the stale base.  A query with
            // every key masked so far keeps m = -inf and gets p = 0 from the -inf scores.
            const float m_cand = fmaxf(m_run, tmax);
            const float m_new = (m_cand - m_run) * sl2 > 8.f ? m_cand : m_run;  // NaN (-inf - -inf): keep
            const float mb = m_new == -INFINITY ? 0.f : m_new * sl2;
            const float corr = exp2_fast(m_run * sl2 - mb);  // 1 when kept; 0 from m_run = -inf
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) s[j][r] = exp2_fast(__builtin_fmaf(s[j][r], sl2, -mb));
            float psum = 0.f;
#pragma unroll
            for (int j = 0; j < NJ; ++j) psum += (s[j][0] + s[j][1]) + (s[j][2] + s[j][3]);
            l_part = l_part * corr + psum;
            m_run = m_new;
            if (__builtin_amdgcn_ballot_w64(corr != 1.0f)) {
                // oacc[c][r] is query 4g + r (O, not O^T), whose factor lives in lane 4g + r,
                // the lane that owns that query's scores
                floatx4 cr;
#pragma unroll
                for (int r = 0; r < 4; ++r) cr[r] = __shfl(corr, 4 * g + r, WAVE);
#pragma unroll
                for (int c = 0; c < NC; ++c) oacc[c] *= cr;
            }
            // O[q][d = 16c + n] += sum_key P[q][key] V[key][d]: in product t of key block j the
            // lanes of group g contribute key 16j + 4g + t -- their own score s[j][t] as A and
            // V[16j + 4g + t][16c + n] as B.  The staged V rows are interleaved (element d at
            // (d % 16) * NC + d / 16), so a lane's NC values for c = 0..NC-1 are adjacent: one
            // 16-byte LDS read per four of them instead of one read per value
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const float *vrow = Vc + (16 * j + 4 * g + t) * KLDV + r16 * NC;
                    float vv[NC];
                    if constexpr (NC % 4 == 0) {
#pragma unroll
                        for (int c = 0; c < NC; c += 4) {
                            const float4 f = *(const float4 *)(vrow + c);
                            vv[c] = f.x, vv[c + 1] = f.y, vv[c + 2] = f.z, vv[c + 3] = f.w;
                        }
                    } else {
#pragma unroll
                        for (int c = 0; c < NC; c += 2) {
                            const float2 f = *(const float2 *)(vrow + c);
                            vv[c] = f.x, vv[c + 1] = f.y;
                        }
                    }
#pragma unroll
                    for (int c = 0; c < NC; ++c) oacc[c] = mfma4(s[j][t], vv[c], oacc[c]);
                }
        }
    };
    // step for tile kv0 in LDS buffer BUF: stage tile kv0+BK from (KR, VR) into the other
    // buffer, refill (KR, VR) with tile kv0+3BK, compute, and wait until every wave is done
    // with buffer BUF before it is restaged
#define FA_STEP(KV0, BUF, KR, VR)                                                            \
    {                                                                                        \
        FA_LSTORE((BUF) ^ 1, KR, VR) /* unused when tile KV0 is the last */                \
        FA_GLOAD(min((KV0) + 3 * BK, k_last), KR, VR)                                        \
        if ((KV0) < wave_kend) tile(KV0, BUF); /* else no tile, or every key masked */       \
        __syncthreads();                                                                     \
    }
    // both steps of an iteration always run (no break between them: a mid-loop exit gives the
    // compiler a path with one register set in flight, and its wait counts then drain both)
    for (int kv0 = k_lo; kv0 < k_end; kv0 += 2 * BK) {
        FA_STEP(kv0, 0, kra, vra)
        FA_STEP(kv0 + BK, 1, krb, vrb)
    }
#undef FA_STEP

    if constexpr (BF16) {
        // O^T accumulators: lane holds O[query = q0 + r16][d = 16c + 4g + r], its own query's
        // row sum in lacc (every entry) and its base in m_run
        if (qi >= p.Sq) return;
        if (p.nsplit > 1) {  // unnormalised partial: O, then the row max (raw units) and row sum
            float *row = p.part + (((long)split * p.B * p.H + bh) * p.Sq + qi) * (D + 2);
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int r = 0; r < 4; ++r) row[16 * c + 4 * g + r] = oacc[c][r];
            if (g == 0) {  // the base in exponent units (-inf: no visible key)
                row[D] = lacc[0] > 0.f ? mb : -INFINITY;
                row[D + 1] = lacc[0];
            }
            return;
        }
        const float inv = lacc[0] > 0.f ? 1.0f / lacc[0] : 0.f;
        const long orow = (long)b * p.o_sb + (long)h * p.o_sh + (long)qi * p.o_ss;
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            uint2 o;
            o.x = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(oacc[c][0] * inv)) |
                  ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(oacc[c][1] * inv)) << 16);
            o.y = (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(oacc[c][2] * inv)) |
                  ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)(oacc[c][3] * inv)) << 16);
            *(uint2 *)((uint16_t *)p.O + orow + 16 * c + 4 * g) = o;
        }
        return;
    } else {
        float l_run = l_part + __shfl_xor(l_part, 16, WAVE);
        l_run += __shfl_xor(l_run, 32, WAVE);
        if (p.nsplit > 1) {  // unnormalised partial: O, then the row max (raw units) and row sum
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float lr = __shfl(l_run, 4 * g + r, WAVE);
                const float mr = __shfl(m_run, 4 * g + r, WAVE);
                const int qo = q0 + 4 * g + r;
                if (qo >= p.Sq) continue;
                float *row = p.part + (((long)split * p.B * p.H + bh) * p.Sq + qo) * (D + 2);
#pragma unroll
                for (int c = 0; c < NC; ++c) row[16 * c + r16] = oacc[c][r];
                if (r16 == 0) {
                    row[D] = mr;
                    row[D + 1] = lr;
                }
            }
            return;
        }
        // lane holds O[query = q0 + 4g + r][d = 16c + r16]; 1/l of query 4g + r from lane 4g + r
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float lr = __shfl(l_run, 4 * g + r, WAVE);
            const int qo = q0 + 4 * g + r;
            if (qo >= p.Sq) continue;
            const float inv = lr > 0.f ? 1.0f / lr : 0.f;
            const long orow = (long)b * p.o_sb + (long)h * p.o_sh + (long)qo * p.o_ss;
#pragma unroll
            for (int c = 0; c < NC; ++c) ((float *)p.O)[orow + 16 * c + r16] = oacc[c][r] * inv;
        }
    }
#undef FA_GLOAD
#undef FA_LSTORE
}

// Combines the key-split partials of a prefill launch: one thread per (row, head-dim
// element); O = sum_i 2^((m_i - M) s) O_i / sum_i 2^((m_i - M) s) l_i with M = max_i m_i
// (s = 1 for bf16 partials, whose m_i are already in exponent units).
template <bool BF16>
__global__ void __launch_bounds__(256) flash_merge_kernel(const PrefillArgs p, int D)
{
    const long g = (long)blockIdx.x * 256 + threadIdx.x;
    const long rows = (long)p.B * p.H * p.Sq;
    if (g >= rows * D) return;
    const long row = g / D;
    const int e = (int)(g % D);
    const int bh = (int)(row / p.Sq), q = (int)(row % p.Sq);
    const long sstride = rows * (D + 2);
    const float *pr = p.part + row * (D + 2);
    float mx = -INFINITY;
    for (int i = 0; i < p.nsplit; ++i) mx = fmaxf(mx, pr[i * sstride + D]);
    float o = 0.f, l = 0.f;
    for (int i = 0; i < p.nsplit; ++i) {
        const float mi = pr[i * sstride + D];
        // bf16 partials carry their base in exponent units, fp32 ones their row max raw
        const float w = mi == -INFINITY ? 0.f : exp2_fast(BF16 ? mi - mx : (mi - mx) * p.scale_log2);
        o += w * pr[i * sstride + e];
        l += w * pr[i * sstride + D + 1];
    }
    const float v = l > 0.f ? o / l : 0.f;
    const int b = bh / p.H, h = bh % p.H;
    const long oi = (long)b * p.o_sb + (long)h * p.o_sh + (long)q * p.o_ss + e;
    if constexpr (BF16)
        ((uint16_t *)p.O)[oi] = __builtin_bit_cast(uint16_t, (__bf16)v);
    else
        ((float *)p.O)[oi] = v;
}

// ---------------------------------------------------------------- decode
struct DecodeArgs {
    const float *q;
    const void *K, *V;  // fp32 or (KB) bf16 elements
    float *O;
    const int32_t *seqlens;
    float *part;    // [B*H][nsplit][D + 2]
    unsigned *ctr;  // [B*H] split-arrival counters, zero between calls
    long k_sb, k_sh;
    int B, H, nsplit, chunk;
    float scale_log2;
    int o_packed_d;  // > 0: write O in the packed B-operand layout over o_packed_d features
};

// Cross-workgroup hand-off of split partials.  The L2 caches of the XCDs are not coherent
// with each other, and a device-scope release or acquire fence writes back or invalidates a
// whole L2 -- per workgroup, far more than the partials.  So the partials are written and
// read with device-scope relaxed atomic stores and loads (coherent across XCDs on their own),
// a wave waits for its stores to complete before the workgroup barrier, and the arrival
// counter is a relaxed atomic add: no fence anywhere.
__device__ __forceinline__ void part_store(float *a, float v)
{
    __hip_atomic_store(a, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float part_load(const float *a)
{
    return __hip_atomic_load(a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Arrival counter of one (sequence, head) pair: the splits that have published their
// partials.  Counter arrays are zero when allocated and the last arrival puts its counter
// back to zero, for the next call and for graph replays.  Returns true for the last arrival.
__device__ __forceinline__ bool decode_arrive(unsigned *ctr, int nsplit)
{
    const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old + 1 != (unsigned)nsplit) return false;
    __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

__device__ __forceinline__ long decode_out_index(const DecodeArgs &p, int bh, int D, int e)
{
    if (p.o_packed_d <= 0) return (long)bh * D + e;
    const int b = bh / p.H, k = (bh % p.H) * D + e;  // token b, feature k
    return ((long)(k >> 4) * 64 + b + 16 * ((k & 15) >> 2)) * 4 + (k & 3);
}

// Sum over the TPK lanes of a key group (TPK = 4, 8, 16 or 32 adjacent lanes), every lane
// receiving the sum, in registers: DPP quad permutes (lane ^ 1, lane ^ 2), then the 8- and
// 16-lane mirrors within a row (each quad, then each half row, meets its partner), then the
// 16-lane row swap across a 32-lane group -- instead of a chain of LDS permutes.  Each step
// adds two values in either order, so all lanes of a group hold the same bits.
template <int TPK>
__device__ __forceinline__ float group_sum(float v)
{
    static_assert(TPK == 4 || TPK == 8 || TPK == 16 || TPK == 32, "key group width");
    auto dpp = [](float x, auto ctrl) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, false));
    };
    v += dpp(v, std::integral_constant<int, 0xB1>{});   // quad_perm [1, 0, 3, 2]
    v += dpp(v, std::integral_constant<int, 0x4E>{});   // quad_perm [2, 3, 0, 1]
    if constexpr (TPK >= 8) v += dpp(v, std::integral_constant<int, 0x141>{});  // row_half_mirror
    if constexpr (TPK >= 16) v += dpp(v, std::integral_constant<int, 0x140>{});  // row_mirror
    if constexpr (TPK >= 32) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    return v;
}

// Merges the nsplit partials (max, sum, weighted values) of pair bh into its output element
// tid.  Eight splits' triples are requested at a time; with at most eight splits the whole
// merge is one memory round trip.  The sums keep split order.
template <int D>
__device__ __forceinline__ void decode_merge_splits(const DecodeArgs &p, int bh, int tid)
{
    const float *pp = p.part + (long)bh * p.nsplit * (D + 2);
    constexpr int G = 8;
    const int ns = p.nsplit;
    float mv[G], lv[G], av[G];
    auto load = [&](int s0) {
#pragma unroll
        for (int u = 0; u < G; ++u) {
            const bool in = s0 + u < ns;
            const float *q = pp + (s0 + u) * (D + 2);
            mv[u] = in ? part_load(q) : -FLT_MAX;
            lv[u] = in ? part_load(q + 1) : 0.f;
            av[u] = in ? part_load(q + 2 + tid) : 0.f;
        }
    };
    load(0);
    float M = -FLT_MAX;
#pragma unroll
    for (int u = 0; u < G; ++u) M = fmaxf(M, mv[u]);
    for (int s0 = G; s0 < ns; ++s0) M = fmaxf(M, part_load(pp + s0 * (D + 2)));
    float L = 0.f, A = 0.f;
    for (int s0 = 0; s0 < ns; s0 += G) {
        if (s0 > 0) load(s0);
#pragma unroll
        for (int u = 0; u < G; ++u) {
            if (s0 + u >= ns) break;
            const float f = mv[u] == -FLT_MAX ? 0.f : exp2f(mv[u] - M);
            L += lv[u] * f;
            A += av[u] * f;
        }
    }
    p.O[decode_out_index(p, bh, D, tid)] = L > 0.f ? A / L : 0.f;
}

// TPK lanes per key (D/4 floats each); each group of TPK lanes walks its own keys.
// KB: the cache holds bf16 keys/values (8-byte loads, widened to fp32).
// WPB waves per workgroup: 4 with key splits; 16 when few (sequence, head) pairs let one
// workgroup take a whole context (no split, no merge launch).
template <int D, bool KB, int WPB>
__global__ void __launch_bounds__(WPB * 64) attn_decode_kernel(const DecodeArgs p)
{
    using KT = typename std::conditional<KB, uint16_t, float>::type;
    constexpr int EPL = KB ? 8 : 4;         // elements per lane and key: one 16-byte load
    constexpr int TPK = D / EPL;            // lanes per key
    constexpr int GPW = WAVE / TPK;         // key groups per wave
    constexpr int NG = WPB * GPW;           // key groups per workgroup
    constexpr int U = WPB > 4 ? 8 : 4;      // keys per group per iteration (loads in flight)
    __shared__ float sm[NG], sl[NG];
    __shared__ float sacc[NG][D];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int grp = w * GPW + lane / TPK, lig = lane % TPK;
    const int bh = blockIdx.y, b = bh / p.H, h = bh % p.H, split = blockIdx.x;
    const int len = p.seqlens[b];
    const int k0 = split * p.chunk, k1 = min(len, k0 + p.chunk);

    float q[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) q[e] = p.q[(long)bh * D + EPL * lig + e] * p.scale_log2;
    const KT *Kb = (const KT *)p.K + (long)b * p.k_sb + (long)h * p.k_sh + EPL * lig;
    const KT *Vb = (const KT *)p.V + (long)b * p.k_sb + (long)h * p.k_sh + EPL * lig;
    // one 16-byte load per key row and lane, kept raw until it is used (bf16: eight elements
    // widened on use, so the registers in flight are the same as for fp32)
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    auto ld16 = [](const KT *a) { return __builtin_nontemporal_load((const u32x4_t *)a); };
    auto elem = [](const u32x4_t &u, int e) -> float {  // element e (compile-time) of a row chunk
        if constexpr (KB) return __uint_as_float(e & 1 ? u[e >> 1] & 0xffff0000u : u[e >> 1] << 16);
        else return __uint_as_float(u[e]);
    };

    float m = -FLT_MAX, l = 0.f;
    float acc[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[e] = 0.f;
    for (int kk = k0 + grp; kk < k1; kk += NG * U) {
        u32x4_t kv[U], vv[U];
        float sc[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            int key = kk + u * NG;
            bool ok = key < k1;
            kv[u] = ok ? ld16(Kb + (long)key * D) : u32x4_t{0u, 0u, 0u, 0u};
            vv[u] = ok ? ld16(Vb + (long)key * D) : u32x4_t{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float d = q[0] * elem(kv[u], 0);
#pragma unroll
            for (int e = 1; e < EPL; ++e) d += q[e] * elem(kv[u], e);
            d = group_sum<TPK>(d);
            sc[u] = (kk + u * NG) < k1 ? d : -FLT_MAX;
        }
        float mx = m;
#pragma unroll
        for (int u = 0; u < U; ++u) mx = fmaxf(mx, sc[u]);
        float corr = exp2f(m - mx);
        l *= corr;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[e] *= corr;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float pv = sc[u] == -FLT_MAX ? 0.f : exp2f(sc[u] - mx);
            l += pv;
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[e] += pv * elem(vv[u], e);
        }
        m = mx;
    }
    // merge the key groups of this workgroup: wave 0 finds the common max and each group's
    // weight (one group per lane, shuffle reductions); then every thread sums the weighted
    // accumulators of a slice of the groups for one output element, and the slices are added
    if (lig == 0) { sm[grp] = m; sl[grp] = l; }
#pragma unroll
    for (int e = 0; e < EPL; e += 4)
        *(float4 *)(&sacc[grp][EPL * lig + e]) = make_float4(acc[e], acc[e + 1], acc[e + 2], acc[e + 3]);
    __syncthreads();
    static_assert(NG <= WAVE, "one key group per lane of wave 0");
    __shared__ float sf[NG], sML[2];
    if (w == 0) {
        const float mg = lane < NG ? sm[lane] : -FLT_MAX;
        const float M = wave_max(mg);
        const float f = (lane < NG && mg != -FLT_MAX) ? exp2f(mg - M) : 0.f;
        const float L = wave_sum(lane < NG ? sl[lane] * f : 0.f);
        if (lane < NG) sf[lane] = f;
        if (lane == 0) { sML[0] = M; sML[1] = L; }
    }
    __syncthreads();
    constexpr int NT = WPB * 64, SL = NT / D < NG ? NT / D : NG;  // slices of the groups
    __shared__ float spart[SL][D];
    if (tid < SL * D) {
        const int sl_i = tid / D, e = tid % D;
        float a = 0.f;
        for (int k = sl_i; k < NG; k += SL) a += sacc[k][e] * sf[k];
        spart[sl_i][e] = a;
    }
    __syncthreads();
    if (tid < D) {
        const float M = sML[0], L = sML[1];
        float A = 0.f;
#pragma unroll
        for (int k = 0; k < SL; ++k) A += spart[k][tid];
        if (p.nsplit == 1) {
            p.O[decode_out_index(p, bh, D, tid)] = L > 0.f ? A / L : 0.f;
        } else {
            float *pp = p.part + ((long)bh * p.nsplit + split) * (D + 2);
            part_store(pp + 2 + tid, A);
            if (tid == 0) { part_store(pp, M); part_store(pp + 1, L); }
        }
    }
    if (p.nsplit == 1) return;
    // the last split of this (sequence, head) to finish merges all of them: every wave's
    // partial stores complete before the barrier, then one arrival is counted
    __shared__ int s_last;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) s_last = decode_arrive(p.ctr + bh, p.nsplit);
    __syncthreads();
    if (!s_last) return;
    if (tid < D) decode_merge_splits<D>(p, bh, tid);
}

// Split count: splits of about 2*B*H keys (at least 192) -- many when few (sequence, head)
// pairs must fill the chip -- but never more than two workgroups per CU need: one split
// when the pairs alone give that (LLaMA-7B at batch 16: 512 pairs, no merge launch).  Then
// max_len is cut into that many equal splits, so no workgroup is left with a short tail
// (1024 + 1024 + 249 keys at 2297 streamed at 6.41 TB/s, 3 x 768 at 6.53).  Measured on
// MI355X: one split against three at 16 x 32 pairs over 2300 keys, 176.7 against 181.7 us
// plus the 4.5 us merge; 4 x 32 pairs, four splits against nine: 47.1 against 49.6 us; batch
// 1 keeps its 12 (16.6 us, the best of 1..24); config 3 (8 x 12 pairs of head dim 64 over 1024
// keys) eight splits of 128 against six of 192: 10.7 against 12.1 us with the merge.  With
// the merge done by each pair's last split (no second launch) config 3 stays at 10.4-10.8 us
// for splits of 64 to 256 keys: the hand-off's store, counter and load round trips cost what
// the merge launch did.  Two tiles of 4 keys in flight per workgroup (the first requested
// together with the query and the length, unpredicated clamped loads) measured no better in
// same-box A/B pairs: config 3 11.5 / 11.3 against 10.6 / 11.2 us, batch-1 LLaMA-7B 197.6
// against 199.0-199.4 tok/s, the batch-16 lines within the run-to-run spread.  A sequence's
// keys fall into the same splits
// for a given max_len (the runner always passes its max_ctx); splits past a shorter
// sequence's length are empty and carry zero weight in the merge.
// bf16 caches take twice the keys per step (8 elements per lane), so their split count is
// never larger than the fp32 one: the fp32 workspace size covers both.
// "wide" form: one 16-wave workgroup per (sequence, head) over the whole context -- no split
// and no merge launch.  It needs few pairs (all of them resident at once) and wins when the
// contexts are short: the decoder runner of a GPT-2 size model (about 500 keys per head at
// 8 x 12 pairs: 0.544 against 0.588 ms per step), but not a full 1024-key cache at the same
// count (18 against 15 us: only 96 CUs stream).  The runner asks for it; jas_attn_decode
// keeps the split form.
// CUs of the current device (256 on MI355X), looked up once per device
static int device_cu_count()
{
    static std::atomic<int> cached[64];  // 0: not looked up yet
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cached[dev].load(std::memory_order_relaxed);
    if (!v) {
        int n = 0;
        v = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0 ? n : 256;
        cached[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

constexpr int DECODE_WIDE_PAIRS = 128;
static bool decode_wide_ok(int B, int H, int D, int max_len, bool kv_bf16)
{
    // a cache of more than 1024 keys per pair keeps the split: one workgroup per pair would
    // stream it from a handful of CUs (LLaMA-7B at batch 1: 32 pairs x 2300 keys)
    return B * H <= DECODE_WIDE_PAIRS && max_len <= 1024 && D >= 64 && !kv_bf16;
}

static int decode_nsplit(int B, int H, int D, int max_len, int *chunk, bool kv_bf16 = false, bool wide = false)
{
    if (wide && decode_wide_ok(B, H, D, max_len, kv_bf16)) {
        *chunk = max_len;
        return 1;
    }
    const int keys_per_step = 4 * (WAVE / (D / (kv_bf16 ? 8 : 4))) * 4;  // NG * U
    // splits of about 2*B*H keys (at least 192), but no more than two workgroups per CU need;
    // head dims up to 64 (half the bytes per key) take splits of B*H keys (at least 128), up
    // to four workgroups per CU
    const bool narrow = D <= 64;
    int ch = narrow ? std::max(B * H, 128) : std::max(2 * B * H, 192);
    ch = (ch + keys_per_step - 1) / keys_per_step * keys_per_step;
    const long pairs = (long)B * H, slots = (narrow ? 4L : 2L) * device_cu_count();
    int ns = std::max(1, (max_len + ch - 1) / ch);
    ns = (int)std::min<long>(ns, std::max(1L, (slots + pairs - 1) / pairs));
    // then equal splits of max_len (e.g. 3 x 768 keys instead of 1024 + 1024 + 249)
    ch = (max_len + ns - 1) / ns;
    ch = (ch + keys_per_step - 1) / keys_per_step * keys_per_step;
    ns = std::max(1, (max_len + ch - 1) / ch);
    *chunk = ch;
    return ns;
}

// the wide form exists for fp32 caches and D >= 64 only (decode_wide_ok)
template <int D>
static void launch_decode_wide(dim3 grid, hipStream_t s, const DecodeArgs &p)
{
    if constexpr (D >= 64) hipLaunchKernelGGL((attn_decode_kernel<D, false, 16>), grid, dim3(1024), 0, s, p);
}

int attn_decode_splits(int B, int H, int D, int max_len, bool kv_bf16, bool wide)
{
    if (B <= 0 || H <= 0 || max_len <= 0 || (D != 32 && D != 64 && D != 128)) return 0;
    int chunk;
    return decode_nsplit(B, H, D, max_len, &chunk, kv_bf16, wide && decode_wide_ok(B, H, D, max_len, kv_bf16));
}

jas_status attn_decode_impl(const float *q, const void *K, const void *V, float *O, const int32_t *seqlens, int B,
                            int H, int D, int max_len, long k_sb, long k_sh, float scale, void *work, unsigned *ctr,
                            hipStream_t s, int o_packed_d, bool kv_bf16, bool wide)
{
    JAS_CHECK(q && K && V && O && seqlens, JAS_ERR_INVALID, "jas_attn_decode: null tensor");
    JAS_CHECK(B > 0 && H > 0 && max_len > 0, JAS_ERR_INVALID, "jas_attn_decode: empty shape");
    JAS_CHECK(D == 32 || D == 64 || D == 128, JAS_ERR_INVALID, "jas_attn_decode: head dim must be 32, 64 or 128");
    JAS_CHECK(k_sb % 4 == 0 && k_sh % 4 == 0, JAS_ERR_INVALID, "jas_attn_decode: strides must be multiples of 4");
    int chunk;
    const bool use_wide = wide && decode_wide_ok(B, H, D, max_len, kv_bf16);
    int ns = decode_nsplit(B, H, D, max_len, &chunk, kv_bf16, use_wide);
    JAS_CHECK(ns == 1 || (work && ctr), JAS_ERR_INVALID, "jas_attn_decode: workspace and counters required");
    JAS_CHECK(o_packed_d <= 0 || (B <= 16 && o_packed_d == H * D), JAS_ERR_INVALID, "attn_decode: bad packed output");
    DecodeArgs p{q, K, V, O, seqlens, (float *)work, ctr, k_sb, k_sh, B, H, ns, chunk, scale * 1.4426950408889634f,
                 o_packed_d};
    dim3 grid(ns, B * H);
#define JAS_DEC(DD)                                                                                  \
    if (D == DD) {                                                                                   \
        if (use_wide) launch_decode_wide<DD>(grid, s, p);                                              \
        else if (kv_bf16) hipLaunchKernelGGL((attn_decode_kernel<DD, true, 4>), grid, dim3(256), 0, s, p); \
        else hipLaunchKernelGGL((attn_decode_kernel<DD, false, 4>), grid, dim3(256), 0, s, p);       \
    }
    JAS_DEC(32) JAS_DEC(64) JAS_DEC(128)
#undef JAS_DEC
    JAS_LAUNCH_CHECK();
    return JAS_OK;
}


// Static scratch of the allocation-free decode entry point: the split partials live in a
// file-scope device array (one copy per GPU, held until the process ends) instead of a
// caller workspace.  Host code never passes the array's name to a kernel (on the host it is
// only a stand-in for the symbol); its device address is looked up once per device with that
// device current and kept here.
static __device__ __align__(256) float scratch[JAS_DECODE_SCRATCH_BYTES / sizeof(float)];
// its split-arrival counters: zero at load, and every call leaves them zero
constexpr int NOALLOC_MAX_PAIRS = 65536;
static __device__ __align__(256) unsigned scratch_arrivals[NOALLOC_MAX_PAIRS];
constexpr int MAX_DEVICES = 64;
static void *scratch_dev_ptr[MAX_DEVICES], *arrivals_dev_ptr[MAX_DEVICES];
static std::mutex scratch_mu;

static jas_status decode_scratch_ptr(void **out, unsigned **ctr)
{
    int dev = 0;
    JAS_HIP(hipGetDevice(&dev));
    JAS_CHECK(dev >= 0 && dev < MAX_DEVICES, JAS_ERR_INVALID, "jas_attn_decode_noalloc: device index out of range");
    std::lock_guard<std::mutex> g(scratch_mu);
    if (!scratch_dev_ptr[dev]) {
        void *ptr = nullptr, *cptr = nullptr;
        JAS_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        JAS_HIP(hipGetSymbolAddress(&cptr, HIP_SYMBOL(scratch_arrivals)));
        JAS_CHECK(ptr && cptr, JAS_ERR_HIP, "jas_attn_decode_noalloc: no device address for the scratch arrays");
        scratch_dev_ptr[dev] = ptr;
        arrivals_dev_ptr[dev] = cptr;
    }
    *out = scratch_dev_ptr[dev];
    *ctr = (unsigned *)arrivals_dev_ptr[dev];
    return JAS_OK;
}

} // namespace jas

using namespace jas;

// fold argument of a causal launch (fa_work_item): the CU count when the kernel's workgroups
// sit exactly two to a CU and the launch has at least two per CU, else 0.  Looked up once per
// kernel and device.
static int fa_fold(const void *kernel, int threads, int total)
{
    static std::mutex mu;
    static std::unordered_map<const void *, int> cache;  // kernel -> workgroups per CU
    int dev = 0, ncu = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    int per = 0;
    {
        std::lock_guard<std::mutex> lk(mu);
        auto it = cache.find(kernel);
        if (it == cache.end()) {
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0) != hipSuccess) per = 0;
            cache.emplace(kernel, per);
        } else {
            per = it->second;
        }
    }
    return per == 2 && ncu % 8 == 0 && total >= 2 * ncu ? ncu : 0;
}

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
    // K/V/Q rows are read in 16-byte chunks (4 f32 / 8 bf16); O is written 4 elements at a time
    const long al = dtype == JAS_BF16 ? 8 : 4;
    JAS_CHECK(q_ss % al == 0 && k_ss % al == 0 && o_ss % al == 0 && q_sh % al == 0 && k_sh % al == 0 &&
                  o_sh % al == 0 && q_sb % al == 0 && k_sb % al == 0 && o_sb % al == 0,
              JAS_ERR_INVALID, "jas_attn_prefill: strides must be multiples of 4 (f32) / 8 (bf16) elements");
    JAS_CHECK((uintptr_t)Q % 16 == 0 && (uintptr_t)K % 16 == 0 && (uintptr_t)V % 16 == 0 && (uintptr_t)O % 16 == 0,
              JAS_ERR_INVALID, "jas_attn_prefill: tensors must be 16-byte aligned");
    PrefillArgs p{Q, K, V, O, q_sb, q_sh, q_ss, k_sb, k_sh, k_ss, o_sb, o_sh, o_ss, B, H, Sq, Sk,
                  scale * 1.4426950408889634f, causal};
    hipStream_t s = stream_or_default(stream);
    // grid: one workgroup per (query block, batch x head), padded to a multiple of the 8 XCDs.
    // When 8-wave workgroups (128 queries) would not give every CU one, 4-wave workgroups
    // (64 queries) double the count -- where a thread's K/V staging stays at four 16-byte
    // loads per tile (not fp32 with D = 128).  A launch that still leaves CUs idle also
    // splits its keys over up to 4 work items (at least two 64-key tiles each), merged by a
    // second kernel; with a causal mask the splits past a query block's diagonal find every
    // key masked and leave a zero-weight partial (decoder self-attention of jasmine's
    // Transformer-base, 8 heads x 512 tokens: forward 0.63 -> 0.57 ms).
    const bool few = (long)ceil_div(Sq, 16 * FA_WAVES) * B * H < 256;
    const int nw = few && (dtype == JAS_BF16 || D <= 64) ? 4 : FA_WAVES;
    const long items = (long)ceil_div(Sq, 16 * nw) * B * H;
    if (items < 256 && Sk >= 4 * 64) {
        int ns = (int)std::min<long>(4, (512 + items - 1) / items);
        ns = std::min(ns, Sk / 128);
        if (ns > 1) {
            p.kchunk = ceil_div(ceil_div(Sk, ns), 64) * 64;
            p.nsplit = ceil_div(Sk, p.kchunk);
            p.part = (float *)workspace(sizeof(float) * (size_t)p.nsplit * B * H * Sq * (D + 2), s);
            JAS_CHECK(p.part, JAS_ERR_OOM, "jas_attn_prefill: workspace allocation failed");
        }
    }
#define JAS_FA_LAUNCH(DD, BF, NWV)                                                                     \
    {                                                                                                  \
        const int total = ceil_div(Sq, 16 * (NWV)) * B * H * p.nsplit;                                 \
        p.fold = causal && p.nsplit == 1 ? fa_fold((const void *)flash_prefill_kernel<DD, BF, 64, NWV>, 64 * (NWV), total) : 0; \
        hipLaunchKernelGGL((flash_prefill_kernel<DD, BF, 64, NWV>), dim3((total + 7) / 8 * 8), dim3(64 * (NWV)), 0, s, p); \
    }
#define JAS_FA(DD)                                                                                     \
    if (D == DD) {                                                                                     \
        if (dtype == JAS_BF16) {                                                                       \
            if (nw == 4) JAS_FA_LAUNCH(DD, true, 4) else JAS_FA_LAUNCH(DD, true, FA_WAVES)             \
        } else {                                                                                       \
            if (nw == 4 && DD <= 64) JAS_FA_LAUNCH(DD, false, 4) else JAS_FA_LAUNCH(DD, false, FA_WAVES) \
        }                                                                                              \
    }
    JAS_FA(32) JAS_FA(64) JAS_FA(128)
#undef JAS_FA
#undef JAS_FA_LAUNCH
    if (p.nsplit > 1) {
        const long n = (long)B * H * Sq * D;
        if (dtype == JAS_BF16) hipLaunchKernelGGL(flash_merge_kernel<true>, dim3(ceil_div(n, 256)), dim3(256), 0, s, p, D);
        else hipLaunchKernelGGL(flash_merge_kernel<false>, dim3(ceil_div(n, 256)), dim3(256), 0, s, p, D);
    }
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
    hipStream_t s = stream_or_default(stream);
    unsigned *ctr = nullptr;
    if (jas_attn_decode_workspace(B, H, D, max_len)) {
        ctr = arrival_counters((size_t)B * H, s);
        JAS_CHECK(ctr, JAS_ERR_OOM, "jas_attn_decode: no memory for the split-arrival counters");
    }
    return attn_decode_impl(q, K, V, O, seqlens, B, H, D, max_len, k_sb, k_sh, scale, work, ctr, s, 0);
}

size_t jas_attn_decode_scratch_max(void) { return JAS_DECODE_SCRATCH_BYTES; }

jas_status jas_attn_decode_noalloc(const float *q, const float *K, const float *V, float *O, const int32_t *seqlens,
                                   int B, int H, int D, int max_len, long k_sb, long k_sh, float scale,
                                   jas_stream_t stream)
{
    const size_t need = jas_attn_decode_workspace(B, H, D, max_len);
    JAS_CHECK(need <= JAS_DECODE_SCRATCH_BYTES, JAS_ERR_INVALID,
              "jas_attn_decode_noalloc: split partials exceed the static scratch (B*H*splits*(D+2)*4 > "
              "jas_attn_decode_scratch_max()); use jas_attn_decode with a workspace");
    void *work = nullptr;
    unsigned *ctr = nullptr;
    if (need) {
        JAS_CHECK((long)B * H <= NOALLOC_MAX_PAIRS, JAS_ERR_INVALID,
                  "jas_attn_decode_noalloc: more than 65536 (sequence, head) pairs with a key split");
        const jas_status st = decode_scratch_ptr(&work, &ctr);
        if (st != JAS_OK) return st;
    }
    return attn_decode_impl(q, K, V, O, seqlens, B, H, D, max_len, k_sb, k_sh, scale, work, ctr,
                            stream_or_default(stream), 0);
}

} // extern "C"
