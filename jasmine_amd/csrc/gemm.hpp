// Internal GEMM entry points shared by the C ABI and the decoder runner.
#pragma once
#include "jas_common.hpp"

namespace jas {

// Fused epilogue of the weight-streaming (decode) GEMM.  Row m of the weight matrix is an
// output feature, column n a token.
enum SkinnyEpi : int {
    EPI_STORE = 0,   // out[n*ldo + m] = act(acc + bias[m])
    EPI_RESID = 1,   // out[n*ldo + m] += acc + bias[m]        (residual stream update)
    EPI_SWIGLU = 2,  // out[n*ldo + m] = silu(acc_gate) * acc_up  (W = gate rows, W2 = up rows)
    EPI_QKV = 3,     // rows [0,d) q, [d,2d) k, [2d,3d) v: (+bias) (+RoPE on q,k), q -> q_out,
                     // k/v -> KV cache at the token's position
    EPI_PARTIAL = 4  // K split over `ksplit` workgroups; out[(s*16 + n)*M + m] = partial sum of
                     // split s (no bias/activation); the consumer adds the splits in order
};

struct SkinnyEpiArgs {
    int mode = EPI_STORE;
    int act = JAS_ACT_NONE;
    const float *bias = nullptr;
    float *out = nullptr;
    long ldo = 0;
    int ksplit = 1;  // EPI_PARTIAL: number of K splits (each gets ceil(chunks/ksplit) 64-chunks)
    int cpb = 0;     // set by skinny_gemm: K chunks per split
    int out_packed = 0;  // EPI_STORE / EPI_SWIGLU: write out in the packed B-operand layout
                         // (packed_b_offset over ldo features) for the next packed GEMM
    // EPI_QKV
    float *q_out = nullptr;   // [n][d]
    float *k_cache = nullptr; // element (n, h, t, e) at n*kv_sb + h*kv_sh + t*dh + e
    float *v_cache = nullptr;
    int kv_bf16 = 0;          // the caches hold bf16 elements (rounded to nearest even)
    const int32_t *pos = nullptr;
    long kv_sb = 0, kv_sh = 0;
    int d = 0, dh = 0;
    int rope = 0;
    float theta = 10000.f;
    // optional [position][dh / 2] (cos, sin) of the rotary angles, the same double values
    // the epilogue would compute; saves the pow / cos / sin at the end of every workgroup
    const double2 *rope_tab = nullptr;
    // EPI_STORE: also the first maximum over this workgroup's rows per token (the LM head's
    // greedy pick), [token][workgroup]; argmax_finish reduces them
    float *amax_v = nullptr;
    int *amax_i = nullptr;
};

// Launch geometry of the weight-streaming GEMM: NT 16-row tiles per workgroup (non-SwiGLU)
// and WPB waves per workgroup splitting K.
struct SkinnyTuning {
    int nt = 1, wpb = 8, depth = 2;  // depth: chunk buffers in the load pipeline
};
SkinnyTuning skinny_default_tuning(int M, int K, bool dual, bool split = false, bool wbf16 = false);
// workgroups along M of a default-tuned launch (the amax_v / amax_i partial count)
int skinny_row_groups(int M, int K, bool dual, bool split = false, bool wbf16 = false);
// K splits (<= 8, all non-empty) for an EPI_PARTIAL launch of an [M][K] weight
int skinny_pick_ksplit(int M, int K, bool wbf16 = false);

// Packed (MFMA-native) weight layout of an [M][K] matrix, rows padded to RG = ceil(M/16)
// row tiles, K % 16 == 0.  A 16 x 16 tile (row tile rt, K block kb) is 256 floats: lane
// l = r%16 + 16*((k%16)/4) holds k%4 = 0..3 -- exactly the A-operand float4 of an MFMA wave,
// one contiguous 1 KB load.  Tiles are ordered CHUNK-MAJOR: K is cut into chunks of 4 blocks
// (64 columns); chunk c holds the tiles (rt, 4c..4c+3) of every row tile, row tile by row
// tile.  Workgroups that stream neighbouring row tiles therefore read neighbouring addresses
// at the same time, which keeps DRAM pages open (a row-tile-major layout, where every
// workgroup streams its own distant range, reaches about half the bandwidth).
__host__ __device__ inline long weight_tile_offset(long rt, int kb, int K16, long RG)
{
    const int c = kb >> 2, q = kb & 3, nb = K16 - 4 * c < 4 ? K16 - 4 * c : 4;  // blocks in chunk c
    return ((long)c * 4 * RG + rt * nb + q) * 256;
}
__host__ __device__ inline long weight_pack_offset(int r, int k, int K, long RG)
{
    const int lane = (r & 15) + 16 * ((k & 15) >> 2);
    return weight_tile_offset(r >> 4, k >> 4, K >> 4, RG) + lane * 4 + (k & 3);
}
__host__ __device__ inline void weight_pack_coords(long p, int K, long RG, int *r, int *k)
{
    const long blk = p >> 8;
    const int within = (int)(p & 255), lane = within >> 2, e = within & 3;
    const int K16 = K >> 4;
    const long c = blk / (4 * RG);  // chunk: full chunks hold 4*RG tiles, the last one fewer
    const int nb = K16 - 4 * (int)c < 4 ? K16 - 4 * (int)c : 4;
    const long in = blk - c * 4 * RG, rt = in / nb;
    const int q = (int)(in - rt * nb);
    *r = (int)(rt * 16 + (lane & 15));
    *k = ((int)c * 4 + q) * 16 + 4 * (lane >> 4) + e;
}
// Packed B-operand (activation) layout of a [16 tokens][K] matrix: element (n, k) at
//   ((k/16) * 64 + lane) * 4 + k%4,  lane = n + 16 * ((k%16)/4)
// so one 16-wide K block is the 64 float4 B-operand registers of an MFMA wave in lane order.
// bf16 packed layout: the same chunk-major order, but the unit is a 16-row x 32-column
// "pair tile" (two 16-wide K blocks, 512 elements, 1 KB) in which lane
// l = r%16 + 16*((k%16)/4) holds 8 consecutive elements, slot 4*((k%32)/16) + k%4 -- exactly
// one lane's operand of a 32-wide v_mfma_f32_16x16x32_bf16 step (with the K order of both
// operands permuted alike), one 16-byte load.  K is padded to a multiple of 32 with zeros;
// a 64-column chunk holds two pair tiles of every row tile (the last chunk one, when the
// padded K is an odd number of pairs).
__host__ __device__ inline int k32_of(int K) { return (K + 31) / 32 * 32; }
__host__ __device__ inline long weight_tile_offset_b(long rt, int kp, int K32, long RG)
{
    const int c = kp >> 1, qp = kp & 1, npairs = K32 >> 5, np = npairs - 2 * c < 2 ? npairs - 2 * c : 2;
    return ((long)c * 2 * RG + rt * np + qp) * 512;
}
__host__ __device__ inline long weight_pack_offset_b(int r, int k, int K, long RG)
{
    const int lane = (r & 15) + 16 * ((k & 15) >> 2), slot = 4 * ((k >> 4) & 1) + (k & 3);
    return weight_tile_offset_b(r >> 4, k >> 5, k32_of(K), RG) + lane * 8 + slot;
}
// inverse over the padded range p < RG*16*K32: (r, k) may be a padding position (k >= K)
__host__ __device__ inline void weight_pack_coords_b(long p, int K, long RG, int *r, int *k)
{
    const long blk = p >> 9;
    const int within = (int)(p & 511), lane = within >> 3, slot = within & 7;
    const int npairs = k32_of(K) >> 5;
    const long c = blk / (2 * RG);
    const int np = npairs - 2 * (int)c < 2 ? npairs - 2 * (int)c : 2;
    const long in = blk - c * 2 * RG, rt = in / np;
    const int qp = (int)(in - rt * np);
    *r = (int)(rt * 16 + (lane & 15));
    *k = ((int)c * 2 + qp) * 32 + 16 * (slot >> 2) + 4 * (lane >> 4) + (slot & 3);
}

__host__ __device__ inline long packed_b_offset(int n, int k)
{
    return ((long)(k >> 4) * 64 + n + 16 * ((k & 15) >> 2)) * 4 + (k & 3);
}
// fp32 row-major [M][K] <-> packed (unpack: packed -> row-major); bf16: the packed side
// holds bf16 elements (packing rounds to nearest even, unpacking widens exactly)
jas_status weight_pack(const void *src, void *dst, int M, int K, bool unpack, hipStream_t s, bool bf16 = false);
jas_status fill_normal_packed(void *x, int M, int K, uint64_t seed, uint64_t stream_id, float mean, float std,
                              hipStream_t s, bool bf16 = false);

// C(n, m) over N <= 16 tokens: acc = W[m, :] . X[n, :].  Row-major: W [M][K], X [N][ldx].
// packed: W in weight_pack_offset layout and X in packed_b_offset layout (ldx ignored).
// W2 (EPI_SWIGLU only) has the same shape and layout as W.
// wbf16 (packed only): W/W2 hold bf16 elements in the packed layout, widened to fp32 on load.
jas_status skinny_gemm(const void *W, const void *W2, const float *X, long ldx, int M, int N, int K,
                       const SkinnyEpiArgs &epi, hipStream_t s, bool packed = false,
                       const SkinnyTuning *tune = nullptr, bool wbf16 = false);

// Fused epilogues of the prefill GEMMs on packed fp32 weights (token-major output).
enum FusedMode : int { FZ_NONE = 0, FZ_QKV = 1, FZ_SWIGLU = 2 };
struct DmaFused {
    int mode = FZ_NONE;
    const float *A2 = nullptr;  // FZ_SWIGLU: the up weights (A: the gate weights)
    // FZ_QKV: rows [0, d) q, [d, 2d) k, [2d, 3d) v; rotary on q and k from rope_tab
    // ([position][dh / 2] (cos, sin)) when rope; k and v also go to the cache at
    // ((seq * H + head) * ctx + pos) * dh, sequence = token / P
    const int32_t *pos = nullptr;
    const double2 *rope_tab = nullptr;
    int rope = 0;
    void *kc = nullptr, *vc = nullptr;
    int kv_bf16 = 0;
    int d = 0, dh = 0, H = 0, P = 0, ctx = 0;
};
// C[n][m] for packed weights A [M][K] and token-major X [N][K], with a fused epilogue;
// false when the product does not qualify (the caller then runs the unfused sequence).
// FZ_SWIGLU: M = 2 x the output features, C [N][M / 2] = silu(gate) * up.
bool gemm_prefill_fused(int M, int N, int K, const void *A, const float *X, float *C, long ldc, const float *bias,
                        const DmaFused &fz, hipStream_t s);

// General strided GEMM (see jas_gemm in jasmine_hip.h).
jas_status gemm_general(int M, int N, int K, const void *A, long as0, long as1, const float *B, long bs0, long bs1,
                        float *C, long cs0, long cs1, const float *bias, int bias_mode, int act, int accumulate,
                        int batch, long abs_, long bbs, long cbs, long biasbs, hipStream_t s, bool a_packed = false,
                        bool a_bf16 = false);

} // namespace jas
