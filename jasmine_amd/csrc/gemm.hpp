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
    EPI_QKV = 3      // rows [0,d) q, [d,2d) k, [2d,3d) v: (+bias) (+RoPE on q,k), q -> q_out,
                     // k/v -> KV cache at the token's position
};

struct SkinnyEpiArgs {
    int mode = EPI_STORE;
    int act = JAS_ACT_NONE;
    const float *bias = nullptr;
    float *out = nullptr;
    long ldo = 0;
    // EPI_QKV
    float *q_out = nullptr;   // [n][d]
    float *k_cache = nullptr; // element (n, h, t, e) at n*kv_sb + h*kv_sh + t*dh + e
    float *v_cache = nullptr;
    const int32_t *pos = nullptr;
    long kv_sb = 0, kv_sh = 0;
    int d = 0, dh = 0;
    int rope = 0;
    float theta = 10000.f;
};

// C(n, m) over N <= 16 tokens: acc = W[m, :] . X[n, :] with W [M][K] and X [N][ldx] both
// K-contiguous.  W2 (EPI_SWIGLU only) has the same shape as W.
jas_status skinny_gemm(const float *W, const float *W2, const float *X, long ldx, int M, int N, int K,
                       const SkinnyEpiArgs &epi, hipStream_t s);

// General strided GEMM (see jas_gemm in jasmine_hip.h).
jas_status gemm_general(int M, int N, int K, const float *A, long as0, long as1, const float *B, long bs0, long bs1,
                        float *C, long cs0, long cs1, const float *bias, int bias_mode, int act, int accumulate,
                        int batch, long abs_, long bbs, long cbs, long biasbs, hipStream_t s);

} // namespace jas
