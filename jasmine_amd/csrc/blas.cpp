// Plain fp32 GEMMs on rocBLAS.
//
// jas_gemm's general form, C = act(A B + bias) (+ C), serves jasmine's mat_dot_t
// (mat_express_t.hpp:696-784) and weight_net_t::forward (mat_net_t.hpp:38-49).  When the
// product is plain (no activation, no bias together with accumulation), large enough to
// amortise the library call, and every operand has a unit stride in one dimension, it goes
// to rocblas_sgemm(_strided_batched): on MI355X that reaches 94 TFLOP/s at 1024^3 and 138 at
// 4096^3 in fp32, against 61-67 and 103 for gemm_tile_kernel.  A bias is then added by a
// small kernel.  Fused epilogues, the decode GEMM and the packed-weight GEMMs of the LM
// runner stay on this library's own kernels.
#include "jas_common.hpp"

#include <mutex>
#include <rocblas/rocblas.h>

namespace jas {
namespace {

std::mutex g_blas_mu;
rocblas_handle g_blas = nullptr;
bool g_blas_failed = false;

// X(r, c) = X[r * s_row + c * s_col] as a column-major rows x cols operand: stored as is
// (unit row stride) or transposed (unit column stride); false when neither applies
bool as_colmajor(long s_row, long s_col, int rows, int cols, rocblas_operation &op, long &ld)
{
    if (s_row == 1 && s_col >= std::max(1, rows)) {
        op = rocblas_operation_none;
        ld = s_col;
        return true;
    }
    if (s_col == 1 && s_row >= std::max(1, cols)) {
        op = rocblas_operation_transpose;
        ld = s_row;
        return true;
    }
    return false;
}

__global__ void add_bias_kernel(float *C, int M, int N, long cs0, long cs1, long cbs, const float *bias, long bbs,
                                int mode)
{
    const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;  // element of batch blockIdx.y
    const long per = (long)M * N;
    if (e >= per) return;
    const int z = blockIdx.y;
    const int m = (int)(e / N), n = (int)(e % N);
    float *c = C + z * cbs + (long)m * cs0 + (long)n * cs1;
    *c += (bias + z * bbs)[mode == 1 ? m : n];
}

} // namespace

// true when the product was issued on rocBLAS (a false return leaves everything to the
// caller); see the conditions above
bool blas_gemm(int M, int N, int K, const float *A, long as0, long as1, const float *B, long bs0, long bs1, float *C,
               long cs0, long cs1, const float *bias, int bias_mode, int act, int accumulate, int batch, long abs_,
               long bbs, long cbs, long biasbs, hipStream_t s)
{
    if (act != JAS_ACT_NONE || (accumulate && bias_mode)) return false;
    if (M < 256 || N < 256 || K < 128) return false;  // small products: the tile kernel
    // column-major C (cs0 == 1): C = A B.  Row-major C (cs1 == 1): C^T = B^T A^T.
    rocblas_operation o1, o2;
    long l1, l2, ldc;
    const float *X1, *X2;
    long x1s, x2s;
    int m, n;
    if (cs0 == 1 && cs1 >= M) {
        if (!as_colmajor(as0, as1, M, K, o1, l1) || !as_colmajor(bs0, bs1, K, N, o2, l2)) return false;
        X1 = A, X2 = B, x1s = abs_, x2s = bbs, m = M, n = N, ldc = cs1;
    } else if (cs1 == 1 && cs0 >= N) {
        if (!as_colmajor(bs1, bs0, N, K, o1, l1) || !as_colmajor(as1, as0, K, M, o2, l2)) return false;
        X1 = B, X2 = A, x1s = bbs, x2s = abs_, m = N, n = M, ldc = cs0;
    } else {
        return false;
    }
    const long lim = 0x7fffffffL;
    if (l1 > lim || l2 > lim || ldc > lim) return false;
    std::lock_guard<std::mutex> lk(g_blas_mu);
    if (g_blas_failed) return false;
    if (!g_blas) {
        // no atomics: every product is summed in a fixed order (run-to-run identical)
        if (rocblas_create_handle(&g_blas) != rocblas_status_success ||
            rocblas_set_atomics_mode(g_blas, rocblas_atomics_not_allowed) != rocblas_status_success) {
            if (g_blas) (void)rocblas_destroy_handle(g_blas);
            g_blas_failed = true;
            g_blas = nullptr;
            return false;
        }
    }
    if (rocblas_set_stream(g_blas, s) != rocblas_status_success) return false;
    const float one = 1.f, beta = accumulate ? 1.f : 0.f;
    rocblas_status st;
    if (batch == 1)
        st = rocblas_sgemm(g_blas, o1, o2, m, n, K, &one, X1, (rocblas_int)l1, X2, (rocblas_int)l2, &beta, C,
                           (rocblas_int)ldc);
    else
        st = rocblas_sgemm_strided_batched(g_blas, o1, o2, m, n, K, &one, X1, (rocblas_int)l1, x1s, X2,
                                           (rocblas_int)l2, x2s, &beta, C, (rocblas_int)ldc, cbs, batch);
    if (st != rocblas_status_success) return false;
    if (bias_mode) {
        const long per = (long)M * N;
        hipLaunchKernelGGL(add_bias_kernel, dim3(ceil_div(per, 256), batch), dim3(256), 0, s, C, M, N, cs0, cs1, cbs,
                           bias, biasbs, bias_mode);
    }
    return true;
}

} // namespace jas
