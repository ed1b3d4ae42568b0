/*
 * oracle.c -- CPU restatement of jasmine's inference arithmetic (see oracle.h).
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, smoke() and bench.py's cpu_baseline leg.
 * Built with -O2 -ffp-contract=off so every float op rounds exactly as written.
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ RNG */
uint64_t orc_splitmix64(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

static uint64_t stream_key(uint64_t seed, uint64_t stream)
{
    return orc_splitmix64(orc_splitmix64(seed) ^ (stream * 0xD1B54A32D192ED03ull));
}

/* Box-Muller on two 53-bit uniforms drawn from counters 2*idx and 2*idx+1. */
static float normal_from_key(uint64_t key, uint64_t idx, float mean, float std)
{
    uint64_t a = orc_splitmix64(key + 2 * idx);
    uint64_t b = orc_splitmix64(key + 2 * idx + 1);
    double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0,1] */
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);         /* [0,1) */
    double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    return (float)((double)mean + (double)std * z);
}

float orc_normal(uint64_t seed, uint64_t stream, uint64_t idx, float mean, float std)
{
    return normal_from_key(stream_key(seed, stream), idx, mean, std);
}

void orc_fill_normal(float *out, size_t n, uint64_t seed, uint64_t stream, float mean, float std)
{
    uint64_t key = stream_key(seed, stream);
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; ++i)
        out[i] = normal_from_key(key, i, mean, std);
}

void orc_fill_randint(int32_t *out, size_t count, uint64_t seed, uint64_t stream, uint32_t n)
{
    uint64_t key = stream_key(seed, stream);
    for (size_t i = 0; i < count; ++i) {
        uint64_t r = orc_splitmix64(key + i) >> 32;
        out[i] = (int32_t)((r * (uint64_t)n) >> 32);
    }
}

/* ------------------------------------------------------------------ L1 */
/* mat_dot_t::operator() (mat_express_t.hpp:730-736): s = 0; s += a*b, k ascending. */
void orc_gemm(int M, int N, int K, const float *A, long as0, long as1,
              const float *B, long bs0, long bs1, float *C, long ldc)
{
#pragma omp parallel for schedule(static) if ((long)M * N * K > (1l << 22))
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float s = 0.0f;
            for (int k = 0; k < K; ++k)
                s += A[i * as0 + k * as1] * B[k * bs0 + j * bs1];
            C[(long)i * ldc + j] = s;
        }
}

/* mat_add_t/mat_sub_t/mat_mul_t work() (mat_express_t.hpp:206-208,270-272,305-307) with
 * ele_type = common_type: (A*B) float, 0.5*C double, sum double, tanh(A) float. */
void orc_cfg2_expr(const float *A, const float *B, const float *C, float *D, size_t n)
{
#pragma omp parallel for schedule(static) if (n > (1u << 20))
    for (size_t i = 0; i < n; ++i) {
        float ab = A[i] * B[i];
        double hc = 0.5 * (double)C[i];
        double s = (double)ab + hc;
        float th = tanhf(A[i]);
        D[i] = (float)(s - (double)th);
    }
}

/* hmax (mat_express_t.hpp:611-628) */
void orc_hmax(const float *X, int R, int C, float *out)
{
    for (int i = 0; i < R; ++i) {
        float m = -FLT_MAX;
        for (int j = 0; j < C; ++j)
            if (X[(long)i * C + j] > m) m = X[(long)i * C + j];
        out[i] = m;
    }
}

/* hsum (mat_express_t.hpp:548-564) */
void orc_hsum(const float *X, int R, int C, float *out)
{
    for (int i = 0; i < R; ++i) {
        float s = 0.0f;
        for (int j = 0; j < C; ++j) s += X[(long)i * C + j];
        out[i] = s;
    }
}

/* vsum (mat_express_t.hpp:530-546) */
void orc_vsum(const float *X, int R, int C, float *out)
{
    for (int j = 0; j < C; ++j) {
        float s = 0.0f;
        for (int i = 0; i < R; ++i) s += X[(long)i * C + j];
        out[j] = s;
    }
}

/* vmean = (vsum / row_num).clone(): float / int -> float (mat_express_t.hpp:566-571) */
void orc_vmean(const float *X, int R, int C, float *out)
{
    orc_vsum(X, R, C, out);
    for (int j = 0; j < C; ++j) out[j] = out[j] / (float)R;
}

/* hmean (mat_express_t.hpp:573-578) */
void orc_hmean(const float *X, int R, int C, float *out)
{
    orc_hsum(X, R, C, out);
    for (int i = 0; i < R; ++i) out[i] = out[i] / (float)C;
}

/* sum (mat_express_t.hpp:518-528): row-major sequential */
float orc_sum(const float *X, int R, int C)
{
    float s = 0.0f;
    for (long i = 0; i < (long)R * C; ++i) s += X[i];
    return s;
}

/* max (mat_express_t.hpp:598-609) */
float orc_max(const float *X, int R, int C)
{
    float m = -FLT_MAX;
    for (long i = 0; i < (long)R * C; ++i)
        if (X[i] > m) m = X[i];
    return m;
}

/* hsoftmax (mat_express_t.hpp:681-694): four materialised float passes. */
void orc_hsoftmax(const float *X, int R, int C, float *Y)
{
#pragma omp parallel for schedule(static) if ((long)R * C > (1l << 20))
    for (int i = 0; i < R; ++i) {
        const float *x = X + (long)i * C;
        float *y = Y + (long)i * C;
        float m = -FLT_MAX;
        for (int j = 0; j < C; ++j)
            if (x[j] > m) m = x[j];
        for (int j = 0; j < C; ++j) y[j] = expf(x[j] - m);
        float s = 0.0f;
        for (int j = 0; j < C; ++j) s += y[j];
        for (int j = 0; j < C; ++j) y[j] = y[j] / s;
    }
}

/* mat_softmax_t (mat_express_t.hpp:642-659): global max, global sum of exp, divide. */
void orc_softmax_global(const float *X, int R, int C, float *Y)
{
    long n = (long)R * C;
    float m = orc_max(X, R, C);
    float s = 0.0f;
    for (long i = 0; i < n; ++i) s += expf(X[i] - m);
    for (long i = 0; i < n; ++i) Y[i] = expf(X[i] - m) / s;
}

/* ------------------------------------------------------------------ L2 */
/* weight_net_t::forward (mat_net_t.hpp:38-49): (W.dot(x) + b).clone(), bias broadcast by
 * modulo over columns (mat_t.hpp:304-305). */
void orc_linear(const float *W, const float *b, const float *X, int out, int in, int T, float *Y)
{
#pragma omp parallel for schedule(static) if ((long)out * in * T > (1l << 22))
    for (int i = 0; i < out; ++i)
        for (int j = 0; j < T; ++j) {
            float s = 0.0f;
            for (int k = 0; k < in; ++k) s += W[(long)i * in + k] * X[(long)k * T + j];
            Y[(long)i * T + j] = s + (b ? b[i] : 0.0f);
        }
}

void orc_relu(const float *X, size_t n, float *Y)
{
    for (size_t i = 0; i < n; ++i) Y[i] = (float)(X[i] > 0) * X[i];
}

/* mat_sigmoid_t::work (mat_express_t.hpp:493-496): exp(-i) on a float is expf, the
 * 1.0 literals then make the rest double. */
void orc_sigmoid(const float *X, size_t n, float *Y)
{
    for (size_t i = 0; i < n; ++i) Y[i] = (float)(1.0 / (1.0 + (double)expf(-X[i])));
}

/* layer_norm_net_t::forward (mat_net_t.hpp:209-225):
 * mean = vmean(x); delta = x - mean; std = sqrt(vmean(pow(delta, 2.0))); hx = delta/std;
 * y = g*hx + b.  pow(float, 2.0) is evaluated in double and stored as float (:587-596). */
void orc_layernorm_cols_jas(const float *X, int R, int C, const float *gamma, const float *beta, float *Y)
{
    for (int j = 0; j < C; ++j) {
        float s = 0.0f;
        for (int i = 0; i < R; ++i) s += X[(long)i * C + j];
        float mean = s / (float)R;
        float s2 = 0.0f;
        for (int i = 0; i < R; ++i) {
            float d = X[(long)i * C + j] - mean;
            s2 += (float)pow((double)d, 2.0);
        }
        float sd = sqrtf(s2 / (float)R);
        for (int i = 0; i < R; ++i) {
            float hx = (X[(long)i * C + j] - mean) / sd;
            float g = gamma ? gamma[i] : 1.0f, bb = beta ? beta[i] : 0.0f;
            Y[(long)i * C + j] = g * hx + bb;
        }
    }
}

void orc_layernorm_rows(const float *X, int R, int C, float eps, const float *g, const float *b, float *Y)
{
#pragma omp parallel for schedule(static) if ((long)R * C > (1l << 20))
    for (int i = 0; i < R; ++i) {
        const float *x = X + (long)i * C;
        float s = 0.0f;
        for (int j = 0; j < C; ++j) s += x[j];
        float mean = s / (float)C;
        float s2 = 0.0f;
        for (int j = 0; j < C; ++j) { float d = x[j] - mean; s2 += d * d; }
        float den = sqrtf(s2 / (float)C + eps);
        for (int j = 0; j < C; ++j)
            Y[(long)i * C + j] = (x[j] - mean) / den * (g ? g[j] : 1.0f) + (b ? b[j] : 0.0f);
    }
}

void orc_rmsnorm_rows(const float *X, int R, int C, float eps, const float *g, float *Y)
{
#pragma omp parallel for schedule(static) if ((long)R * C > (1l << 20))
    for (int i = 0; i < R; ++i) {
        const float *x = X + (long)i * C;
        float s2 = 0.0f;
        for (int j = 0; j < C; ++j) s2 += x[j] * x[j];
        float den = sqrtf(s2 / (float)C + eps);
        for (int j = 0; j < C; ++j) Y[(long)i * C + j] = x[j] / den * (g ? g[j] : 1.0f);
    }
}

float orc_gelu(float x)
{
    double v = (double)x;
    return (float)(0.5 * v * (1.0 + tanh(0.7978845608028654 * (v + 0.044715 * v * v * v))));
}

float orc_silu(float x)
{
    double v = (double)x;
    return (float)(v / (1.0 + exp(-v)));
}

/* ------------------------------------------------------------------ L3 */
/* mat_head_gen_t::forward (mat_mha_t.hpp:45-74; cross form :76-90). */
void orc_jas_head(const float *Xq, const float *Xkv, int dh, int Tq, int Tk,
                  const float *Wq, const float *bq, const float *Wk, const float *bk,
                  const float *Wv, const float *bv, int mask, float *Y)
{
    float *q = malloc(sizeof(float) * dh * Tq);
    float *k = malloc(sizeof(float) * dh * Tk);
    float *v = malloc(sizeof(float) * dh * Tk);
    float *S = malloc(sizeof(float) * Tq * Tk);
    float *P = malloc(sizeof(float) * Tq * Tk);
    orc_linear(Wq, bq, Xq, dh, dh, Tq, q);
    orc_linear(Wk, bk, Xkv, dh, dh, Tk, k);
    orc_linear(Wv, bv, Xkv, dh, dh, Tk, v);
    double sq = sqrt((double)dh);  /* sqrt(int) -> double (mat_mha_t.hpp:53) */
    for (int i = 0; i < Tq; ++i)
        for (int j = 0; j < Tk; ++j) {
            float s = 0.0f;  /* m_q.t().dot(m_k): sum over feature rows */
            for (int r = 0; r < dh; ++r) s += q[r * Tq + i] * k[r * Tk + j];
            S[i * Tk + j] = (float)((double)s / sq);  /* mat_t<double> -> mat_t<float> */
            if (mask && j > i) S[i * Tk + j] = -INFINITY;  /* mat_mha_t.hpp:58-67 */
        }
    orc_hsoftmax(S, Tq, Tk, P);
    /* m_v.dot(attn_weights.t()) (mat_mha_t.hpp:71) */
    for (int r = 0; r < dh; ++r)
        for (int i = 0; i < Tq; ++i) {
            float s = 0.0f;
            for (int j = 0; j < Tk; ++j) s += v[r * Tk + j] * P[i * Tk + j];
            Y[r * Tq + i] = s;
        }
    free(q); free(k); free(v); free(S); free(P);
}

size_t orc_jas_mha_nparams(int d, int H)
{
    size_t dh = (size_t)(d / H);
    return (size_t)H * 3 * (dh * dh + dh) + (size_t)d * d + d;
}

/* mat_mha_t::forward (mat_mha_t.hpp:265-291 self, 293-322 cross) */
void orc_jas_mha(const float *Xq, const float *Xkv, int d, int H, int Tq, int Tk,
                 const float *W, int mask, float *Y)
{
    int dh = d / H;
    float *cat = malloc(sizeof(float) * d * Tq);
    const float *p = W;
    for (int h = 0; h < H; ++h) {
        const float *Wq = p, *bq = p + dh * dh; p += dh * dh + dh;
        const float *Wk = p, *bk = p + dh * dh; p += dh * dh + dh;
        const float *Wv = p, *bv = p + dh * dh; p += dh * dh + dh;
        /* vsplit: rows [h*dh, (h+1)*dh) of the [d,T] input (mat_mha_t.hpp:198-215) */
        orc_jas_head(Xq + (long)h * dh * Tq, Xkv + (long)h * dh * Tk, dh, Tq, Tk,
                     Wq, bq, Wk, bk, Wv, bv, mask, cat + (long)h * dh * Tq);
    }
    orc_linear(p, p + (long)d * d, cat, d, d, Tq, Y);
    free(cat);
}

/* double-precision ground truth attention, [B,H,S,D] */
void orc_attention(const float *Q, const float *K, const float *V, float *O,
                   int B, int H, int Sq, int Sk, int D, double scale, int causal)
{
#pragma omp parallel for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const float *q = Q + ((long)(b * H + h) * Sq) * D;
            const float *k = K + ((long)(b * H + h) * Sk) * D;
            const float *v = V + ((long)(b * H + h) * Sk) * D;
            float *o = O + ((long)(b * H + h) * Sq) * D;
            double *s = malloc(sizeof(double) * Sk);
            double *acc = malloc(sizeof(double) * D);
            for (int i = 0; i < Sq; ++i) {
                int lim = causal ? i + Sk - Sq : Sk - 1;
                double m = -INFINITY;
                for (int j = 0; j <= lim; ++j) {
                    double t = 0.0;
                    for (int e = 0; e < D; ++e) t += (double)q[(long)i * D + e] * (double)k[(long)j * D + e];
                    s[j] = t * scale;
                    if (s[j] > m) m = s[j];
                }
                double l = 0.0;
                for (int e = 0; e < D; ++e) acc[e] = 0.0;
                for (int j = 0; j <= lim; ++j) {
                    double p = exp(s[j] - m);
                    l += p;
                    for (int e = 0; e < D; ++e) acc[e] += p * (double)v[(long)j * D + e];
                }
                for (int e = 0; e < D; ++e) o[(long)i * D + e] = (float)(acc[e] / l);
            }
            free(s); free(acc);
        }
}

/* ------------------------------------------------------------------ RoPE */
/* cache entry (r, c) of mat_RoPE_t::init (mat_RoPE_t.hpp:107-131) for val_type float:
 * angle = (float)(c / pow(10000.0, (float)(r/2) / (float)d)); cos on the diagonal parity,
 * -sin at (even, odd), sin at (odd, even). */
static float rope_jas_entry(int r, int c, int d)
{
    float e = (float)(r / 2) / (float)d;
    float angle = (float)((double)c / pow(10000.0, (double)e));
    if ((r % 2) == (c % 2)) return cosf(angle);
    if (r % 2 == 0) return -sinf(angle);
    return sinf(angle);
}

/* RoPE_net_t::forward (mat_RoPE_t.hpp:166-188): per (m, i) the 2x2 block at cache rows
 * 2i..2i+1, cols 2m..2m+1 times the 2x1 input slice, float dot. */
void orc_rope_jas(const float *X, int d, int T, float *Y)
{
    for (int m = 0; m < T; ++m)
        for (int i = 0; i < d / 2; ++i) {
            float x0 = X[(2 * i) * T + m], x1 = X[(2 * i + 1) * T + m];
            for (int r = 0; r < 2; ++r) {
                float s = 0.0f;
                s += rope_jas_entry(2 * i + r, 2 * m, d) * x0;
                s += rope_jas_entry(2 * i + r, 2 * m + 1, d) * x1;
                Y[(2 * i + r) * T + m] = s;
            }
        }
    if (d % 2) /* odd trailing row is left as zero by jasmine (ret is zero-initialised) */
        for (int m = 0; m < T; ++m) Y[(d - 1) * T + m] = 0.0f;
}

void orc_rope_llama(float *x, int dh, int pos, float theta)
{
    for (int i = 0; i < dh / 2; ++i) {
        double inv = pow((double)theta, -2.0 * i / (double)dh);
        double a = (double)pos * inv;
        double c = cos(a), s = sin(a);
        double x0 = x[2 * i], x1 = x[2 * i + 1];
        x[2 * i] = (float)(x0 * c - x1 * s);
        x[2 * i + 1] = (float)(x0 * s + x1 * c);
    }
}

/* ------------------------------------------------------------------ L4 stacks */
static size_t ffn_nparams(int d) { return (size_t)d * d + d; }

size_t orc_jas_encoder_layer_nparams(int d, int H)
{
    return orc_jas_mha_nparams(d, H) + ffn_nparams(d);
}

size_t orc_jas_decoder_layer_nparams(int d, int H)
{
    return 2 * orc_jas_mha_nparams(d, H) + ffn_nparams(d);
}

/* residual_net_t::forward (mat_net_t.hpp:326-329) then layer_norm_net_t (defaults 1/0) */
static void add_ln(float *X, const float *R, int d, int T)
{
    for (long i = 0; i < (long)d * T; ++i) X[i] = R[i] + X[i];
    float *tmp = malloc(sizeof(float) * d * T);
    orc_layernorm_cols_jas(X, d, T, NULL, NULL, tmp);
    memcpy(X, tmp, sizeof(float) * d * T);
    free(tmp);
}

/* res_ffn_t: relu(W x + b) + x (mat_transformer_kernel_t.hpp:26-33) */
static void ffn_block(float *X, const float *W, int d, int T)
{
    float *t = malloc(sizeof(float) * d * T);
    orc_linear(W, W + (long)d * d, X, d, d, T, t);
    orc_relu(t, (size_t)d * T, t);
    add_ln(t, X, d, T); /* t = LN(relu(.) + x) */
    memcpy(X, t, sizeof(float) * d * T);
    free(t);
}

void orc_jas_encoder_layer(const float *X, int d, int H, int T, const float *W, float *Y)
{
    float *a = malloc(sizeof(float) * d * T);
    memcpy(Y, X, sizeof(float) * d * T);
    orc_jas_mha(Y, Y, d, H, T, T, W, 0, a);
    add_ln(a, Y, d, T);
    memcpy(Y, a, sizeof(float) * d * T);
    ffn_block(Y, W + orc_jas_mha_nparams(d, H), d, T);
    free(a);
}

void orc_jas_decoder_layer(const float *X, const float *enc, int d, int H, int T, int Te,
                           const float *W, float *Y)
{
    float *a = malloc(sizeof(float) * d * T);
    size_t nm = orc_jas_mha_nparams(d, H);
    memcpy(Y, X, sizeof(float) * d * T);
    orc_jas_mha(Y, Y, d, H, T, T, W, 1, a);
    add_ln(a, Y, d, T);
    memcpy(Y, a, sizeof(float) * d * T);
    orc_jas_mha(Y, enc, d, H, T, Te, W + nm, 0, a);
    add_ln(a, Y, d, T);
    memcpy(Y, a, sizeof(float) * d * T);
    ffn_block(Y, W + 2 * nm, d, T);
    free(a);
}

void orc_jas_transformer(const float *en, int Te, const float *de, int Td, int d, int H,
                         int n_enc, int n_dec, const float *W, float *Y)
{
    float *e = malloc(sizeof(float) * d * Te);
    float *t = malloc(sizeof(float) * d * (Te > Td ? Te : Td));
    orc_rope_jas(en, d, Te, e);
    const float *p = W;
    for (int l = 0; l < n_enc; ++l) {
        orc_jas_encoder_layer(e, d, H, Te, p, t);
        memcpy(e, t, sizeof(float) * d * Te);
        p += orc_jas_encoder_layer_nparams(d, H);
    }
    orc_rope_jas(de, d, Td, Y);
    for (int l = 0; l < n_dec; ++l) {
        orc_jas_decoder_layer(Y, e, d, H, Td, Te, p, t);
        memcpy(Y, t, sizeof(float) * d * Td);
        p += orc_jas_decoder_layer_nparams(d, H);
    }
    free(e); free(t);
}

/* ------------------------------------------------------------------ decoder LMs */
int orc_argmax(const float *x, int n)
{
    int best = 0;
    for (int i = 1; i < n; ++i)
        if (x[i] > x[best]) best = i;
    return best;
}

/* y[out] = W[out][in] . x[in] (+ b), float sequential k.  Rows are independent, so they
 * are spread over threads when the caller is not already parallel (one sequence). */
static void matvec(const float *W, const float *b, const float *x, int out, int in, float *y)
{
#pragma omp parallel for schedule(static) if (!omp_in_parallel() && (long)out * in > (1l << 20))
    for (int i = 0; i < out; ++i) {
        const float *w = W + (long)i * in;
        float s = 0.0f;
        for (int k = 0; k < in; ++k) s += w[k] * x[k];
        y[i] = b ? s + b[i] : s;
    }
}

typedef struct {
    const orc_lm_cfg *c;
    const orc_lm_weights *w;
    float *kc, *vc; /* [B][L][H][ctx][dh] */
} lm_state;

static float *kv_at(const lm_state *st, float *base, int b, int l, int h, int t)
{
    const orc_lm_cfg *c = st->c;
    int dh = c->d_model / c->n_head;
    return base + ((((long)b * c->n_layer + l) * c->n_head + h) * c->max_ctx + t) * dh;
}

/* fp32 -> bf16 -> fp32, round to nearest even (the cache element of a bf16 KV cache) */
static float round_bf16(float f)
{
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return f;
    u = ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) << 16;
    memcpy(&f, &u, 4);
    return f;
}

/* Round every cached key/value of sequence b at positions [0, n) (bf16 KV cache). */
static void lm_round_cache(const lm_state *st, int b, int n)
{
    const orc_lm_cfg *c = st->c;
    int dh = c->d_model / c->n_head;
    for (int l = 0; l < c->n_layer; ++l)
        for (int h = 0; h < c->n_head; ++h)
            for (int t = 0; t < n; ++t) {
                float *k = kv_at(st, st->kc, b, l, h, t), *v = kv_at(st, st->vc, b, l, h, t);
                for (int e = 0; e < dh; ++e) { k[e] = round_bf16(k[e]); v[e] = round_bf16(v[e]); }
            }
}

/* Process token `tok` at position `pos` of sequence b through all layers, attending to
 * cache entries 0..pos; writes final-norm hidden into hout[d].  round_new: the token's own
 * key/value enter the cache rounded to bf16 (a generated token under a bf16 KV cache). */
static void lm_token(const lm_state *st, int b, int tok, int pos, float *hout, int round_new)
{
    const orc_lm_cfg *c = st->c;
    const orc_lm_weights *w = st->w;
    int d = c->d_model, H = c->n_head, dh = d / H, F = c->d_ff;
    float *x = malloc(sizeof(float) * d), *h = malloc(sizeof(float) * d);
    float *qkv = malloc(sizeof(float) * 3 * d), *att = malloc(sizeof(float) * d);
    float *t1 = malloc(sizeof(float) * F), *t2 = malloc(sizeof(float) * F);
    float *o = malloc(sizeof(float) * d);
    double *sc = malloc(sizeof(double) * (pos + 1));
    for (int i = 0; i < d; ++i)
        x[i] = c->kind == 0 ? w->wte[(long)tok * d + i] + w->wpe[(long)pos * d + i]
                            : w->wte[(long)tok * d + i];
    for (int l = 0; l < c->n_layer; ++l) {
        if (c->kind == 0)
            orc_layernorm_rows(x, 1, d, c->eps, w->ln1_g + (long)l * d, w->ln1_b + (long)l * d, h);
        else
            orc_rmsnorm_rows(x, 1, d, c->eps, w->ln1_g + (long)l * d, h);
        matvec(w->w_qkv + (long)l * 3 * d * d, w->b_qkv ? w->b_qkv + (long)l * 3 * d : NULL, h, 3 * d, d, qkv);
        for (int hh = 0; hh < H; ++hh) {
            float *q = qkv + hh * dh, *k = qkv + d + hh * dh, *v = qkv + 2 * d + hh * dh;
            if (c->kind == 1) {
                orc_rope_llama(q, dh, pos, c->rope_theta);
                orc_rope_llama(k, dh, pos, c->rope_theta);
            }
            float *kd = kv_at(st, st->kc, b, l, hh, pos), *vd = kv_at(st, st->vc, b, l, hh, pos);
            for (int e = 0; e < dh; ++e) {
                kd[e] = round_new ? round_bf16(k[e]) : k[e];
                vd[e] = round_new ? round_bf16(v[e]) : v[e];
            }
            double scale = 1.0 / sqrt((double)dh), m = -INFINITY;
            for (int t = 0; t <= pos; ++t) {
                const float *kt = kv_at(st, st->kc, b, l, hh, t);
                double s = 0.0;
                for (int e = 0; e < dh; ++e) s += (double)q[e] * (double)kt[e];
                sc[t] = s * scale;
                if (sc[t] > m) m = sc[t];
            }
            double lsum = 0.0;
            for (int t = 0; t <= pos; ++t) { sc[t] = exp(sc[t] - m); lsum += sc[t]; }
            for (int e = 0; e < dh; ++e) {
                double a = 0.0;
                for (int t = 0; t <= pos; ++t) a += sc[t] * (double)kv_at(st, st->vc, b, l, hh, t)[e];
                att[hh * dh + e] = (float)(a / lsum);
            }
        }
        matvec(w->w_o + (long)l * d * d, w->b_o ? w->b_o + (long)l * d : NULL, att, d, d, o);
        for (int i = 0; i < d; ++i) x[i] = x[i] + o[i];
        if (c->kind == 0) {
            orc_layernorm_rows(x, 1, d, c->eps, w->ln2_g + (long)l * d, w->ln2_b + (long)l * d, h);
            matvec(w->w_fc + (long)l * F * d, w->b_fc + (long)l * F, h, F, d, t1);
            for (int i = 0; i < F; ++i) t1[i] = orc_gelu(t1[i]);
            matvec(w->w_proj + (long)l * d * F, w->b_proj + (long)l * d, t1, d, F, o);
        } else {
            orc_rmsnorm_rows(x, 1, d, c->eps, w->ln2_g + (long)l * d, h);
            matvec(w->w_gate + (long)l * F * d, NULL, h, F, d, t1);
            matvec(w->w_up + (long)l * F * d, NULL, h, F, d, t2);
            for (int i = 0; i < F; ++i) t1[i] = orc_silu(t1[i]) * t2[i];
            matvec(w->w_down + (long)l * d * F, NULL, t1, d, F, o);
        }
        for (int i = 0; i < d; ++i) x[i] = x[i] + o[i];
    }
    if (c->kind == 0)
        orc_layernorm_rows(x, 1, d, c->eps, w->lnf_g, w->lnf_b, hout);
    else
        orc_rmsnorm_rows(x, 1, d, c->eps, w->lnf_g, hout);
    free(x); free(h); free(qkv); free(att); free(t1); free(t2); free(o); free(sc);
}

static void lm_logits(const lm_state *st, const float *hf, float *logits)
{
    const orc_lm_cfg *c = st->c;
    const float *head = c->kind == 0 ? st->w->wte : st->w->w_head;
    matvec(head, NULL, hf, c->vocab, c->d_model, logits);
}

void orc_lm_generate(const orc_lm_cfg *cfg, const orc_lm_weights *w, int B, int P,
                     const int32_t *prompt, int steps, const int32_t *force_ids,
                     int32_t *out_ids, float *logits, int nthreads)
{
    int d = cfg->d_model, V = cfg->vocab;
    long kvn = (long)B * cfg->n_layer * cfg->n_head * cfg->max_ctx * (d / cfg->n_head);
    lm_state st = {cfg, w, calloc(kvn, sizeof(float)), calloc(kvn, sizeof(float))};
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
#pragma omp parallel for schedule(dynamic) if (B > 1)
    for (int b = 0; b < B; ++b) {
        float *hf = malloc(sizeof(float) * d), *lg = malloc(sizeof(float) * V);
        for (int t = 0; t < P - 1; ++t) lm_token(&st, b, prompt[(long)b * P + t], t, hf, 0);
        int tok = prompt[(long)b * P + P - 1];
        for (int s = 0; s < steps; ++s) {
            /* step 0 is the prompt's last token: part of the prefill */
            lm_token(&st, b, tok, P - 1 + s, hf, s > 0 && cfg->kv_bf16);
            if (s == 0 && cfg->kv_bf16) lm_round_cache(&st, b, P);
            lm_logits(&st, hf, lg);
            int nx = orc_argmax(lg, V);
            out_ids[(long)b * steps + s] = nx;
            if (logits) memcpy(logits + ((long)s * B + b) * V, lg, sizeof(float) * V);
            tok = force_ids ? force_ids[(long)b * steps + s] : nx;
        }
        free(hf); free(lg);
    }
    free(st.kc); free(st.vc);
}

void orc_lm_last_logits(const orc_lm_cfg *cfg, const orc_lm_weights *w, int B, int T,
                        const int32_t *ids, float *logits, int nthreads)
{
    int d = cfg->d_model;
    long kvn = (long)B * cfg->n_layer * cfg->n_head * cfg->max_ctx * (d / cfg->n_head);
    lm_state st = {cfg, w, calloc(kvn, sizeof(float)), calloc(kvn, sizeof(float))};
#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
#pragma omp parallel for schedule(dynamic) if (B > 1)
    for (int b = 0; b < B; ++b) {
        float *hf = malloc(sizeof(float) * d);
        for (int t = 0; t < T; ++t) lm_token(&st, b, ids[(long)b * T + t], t, hf, 0);
        lm_logits(&st, hf, logits + (long)b * cfg->vocab);
        free(hf);
    }
    free(st.kc); free(st.vc);
}
