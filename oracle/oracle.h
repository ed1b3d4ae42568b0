/*
 * oracle.h -- CPU restatement of jasmine's transformer inference arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load liboracle.so, and only as the checker
 * (or the timed CPU baseline).  The product library (libjasmine_hip.so) never
 * links or calls anything here.
 *
 * Every function states the reference code it restates (file:line into the
 * jasmine sources).  Arithmetic order and precision follow jasmine exactly:
 *   - matrix products accumulate sequentially in k, in the element type,
 *     starting from 0 (mat_express_t.hpp:730-736), no fused multiply-add;
 *   - scalar operands promote through std::common_type (a double scalar makes
 *     the node double, mat_express_t.hpp:20-24,44);
 *   - row/column sums are sequential (mat_express_t.hpp:511-564).
 * Ops jasmine lacks (tanh, GELU, RMSNorm, SwiGLU, LLaMA RoPE, embeddings,
 * KV cache, argmax) are restated from their textbook closed forms; their
 * pinning is listed in the oracle test file header.
 *
 * Layout: all matrices are dense row-major float32 unless stated.
 */
#ifndef JASMINE_ORACLE_H
#define JASMINE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------- portable random numbers (shared by GPU weight init) ---------- */
uint64_t orc_splitmix64(uint64_t x);
/* N(mean, std) for element idx of stream (seed, stream): counter based. */
float orc_normal(uint64_t seed, uint64_t stream, uint64_t idx, float mean, float std);
void orc_fill_normal(float *out, size_t n, uint64_t seed, uint64_t stream, float mean, float std);
/* uniform integers in [0, n) (Lemire multiply-shift on the top 32 bits). */
void orc_fill_randint(int32_t *out, size_t count, uint64_t seed, uint64_t stream, uint32_t n);

/* ---------- L1: expression engine ---------- */
/* C[M,N] = A[M,K] . B[K,N]   (mat_dot_t, mat_express_t.hpp:730-736)
 * generic strides so transposed views can be expressed: A(i,k) = A[i*as0 + k*as1]. */
void orc_gemm(int M, int N, int K, const float *A, long as0, long as1,
              const float *B, long bs0, long bs1, float *C, long ldc);
/* D = A*B + 0.5*C - tanh(A) with jasmine promotion: the 0.5 scalar makes the sum
 * double (mat_express_t.hpp:20-24,44); A*B and tanh(A) are float nodes. */
void orc_cfg2_expr(const float *A, const float *B, const float *C, float *D, size_t n);
/* row softmax: hmax, exp(x - max), hsum, divide (mat_express_t.hpp:681-694) */
void orc_hsoftmax(const float *X, int R, int C, float *Y);
/* whole-matrix softmax mat_softmax_t (mat_express_t.hpp:630-665) */
void orc_softmax_global(const float *X, int R, int C, float *Y);
/* hsum/vsum/hmax/vmean/hmean/sum/max (mat_express_t.hpp:511-628) */
void orc_hsum(const float *X, int R, int C, float *out /*R*/);
void orc_vsum(const float *X, int R, int C, float *out /*C*/);
void orc_hmax(const float *X, int R, int C, float *out /*R*/);
void orc_vmean(const float *X, int R, int C, float *out /*C*/);
void orc_hmean(const float *X, int R, int C, float *out /*R*/);
float orc_sum(const float *X, int R, int C);
float orc_max(const float *X, int R, int C);

/* ---------- L2: layers ---------- */
/* Y[out,T] = W[out,in] . X[in,T] + b[out]  (weight_net_t::forward, mat_net_t.hpp:38-49) */
void orc_linear(const float *W, const float *b, const float *X, int out, int in, int T, float *Y);
/* (x > 0) * x   (relu_net_t::forward, mat_net_t.hpp:146-153): bool promoted to float then
 * multiplied, so negative x gives -0.0f and -inf gives NaN exactly as jasmine. */
void orc_relu(const float *X, size_t n, float *Y);
/* 1.0/(1.0+expf(-x)): expf in float, the rest in double (mat_express_t.hpp:493-496) */
void orc_sigmoid(const float *X, size_t n, float *Y);
/* column LayerNorm, population std, NO eps (layer_norm_net_t::forward mat_net_t.hpp:209-225)
 * gamma/beta are per-row [R]; pass NULL for the lazily-created 1/0 defaults. */
void orc_layernorm_cols_jas(const float *X, int R, int C, const float *gamma, const float *beta, float *Y);
/* row LayerNorm with eps (config 2): y = (x - mean)/sqrt(var + eps) * g + b, float sums. */
void orc_layernorm_rows(const float *X, int R, int C, float eps, const float *g, const float *b, float *Y);
/* row RMSNorm (config 2 / LLaMA): y = x / sqrt(mean(x^2) + eps) * g */
void orc_rmsnorm_rows(const float *X, int R, int C, float eps, const float *g, float *Y);
/* GPT-2 GELU, tanh form, evaluated in double and rounded */
float orc_gelu(float x);
float orc_silu(float x);

/* ---------- L3: attention ---------- */
/* one jasmine head (mat_head_gen_t::forward, mat_mha_t.hpp:45-74 self / 76-90 cross):
 * Xq[dh,Tq], Xkv[dh,Tk] feature-major; W* [dh,dh]; b* [dh]; Y[dh,Tq].
 * score = (float)((double)dot_f / sqrt((double)dh)), causal mask j>i -> -inf. */
void orc_jas_head(const float *Xq, const float *Xkv, int dh, int Tq, int Tk,
                  const float *Wq, const float *bq, const float *Wk, const float *bk,
                  const float *Wv, const float *bv, int mask, float *Y);
/* mat_mha_t::forward (mat_mha_t.hpp:265-322): block-diagonal heads over row slices,
 * vconcat, output projection.  W packs per head [Wq,bq,Wk,bk,Wv,bv] then [Wo,bo]
 * in jasmine init_weight traversal order (mat_mha_t.hpp:384-392). */
size_t orc_jas_mha_nparams(int d, int H);
void orc_jas_mha(const float *Xq, const float *Xkv, int d, int H, int Tq, int Tk,
                 const float *W, int mask, float *Y);
/* standard scaled-dot attention, token-major Q[B,H,Sq,D], K/V[B,H,Sk,D] -> O; computed in
 * double (ground truth for flash prefill / split-K decode).  Causal aligns the last query
 * with the last key (query i sees keys j <= i + Sk - Sq). */
void orc_attention(const float *Q, const float *K, const float *V, float *O,
                   int B, int H, int Sq, int Sk, int D, double scale, int causal);

/* ---------- RoPE ---------- */
/* jasmine RoPE_net_t::forward (mat_RoPE_t.hpp:166-188) with the cache angles of
 * mat_RoPE_t::init (mat_RoPE_t.hpp:107-131): X[d,T] feature-major */
void orc_rope_jas(const float *X, int d, int T, float *Y);
/* LLaMA rotary on interleaved pairs of one head vector x[dh] at position pos. */
void orc_rope_llama(float *x, int dh, int pos, float theta);

/* ---------- L4/L5: jasmine post-LN stacks (mat_transformer_kernel_t.hpp) ---------- */
/* parameter counts in jasmine init_weight traversal order */
size_t orc_jas_encoder_layer_nparams(int d, int H);
size_t orc_jas_decoder_layer_nparams(int d, int H);
/* encoder layer: LN(x + MHA(x)) then LN(. + relu(W . + b))  (mat_transformer_kernel_t.hpp:41-45) */
void orc_jas_encoder_layer(const float *X, int d, int H, int T, const float *W, float *Y);
/* decoder layer: masked MHA, cross MHA on enc[d,Te], FFN, each residual+LN
 * (mat_transformer_kernel_t.hpp:47-52) */
void orc_jas_decoder_layer(const float *X, const float *enc, int d, int H, int T, int Te,
                           const float *W, float *Y);
/* transformer_base_t: encoder_forward(en) then forward(de) (mat_transformer_t.hpp:36-44).
 * W = [encoder layers..., decoder layers...] */
void orc_jas_transformer(const float *en, int Te, const float *de, int Td, int d, int H,
                         int n_enc, int n_dec, const float *W, float *Y);

/* ---------- decoder-only LMs (GPT-2 / LLaMA shapes, build's own composition) ---------- */
typedef struct {
    int kind;        /* 0 = GPT-2 (pre-LN, GELU, learned pos, tied head), 1 = LLaMA */
    int n_layer, d_model, n_head, d_ff, vocab, max_ctx;
    float eps;       /* 1e-5 GPT-2 LN, 1e-6 LLaMA RMSNorm */
    float rope_theta;
    /* 1: the KV cache stores keys/values rounded to bf16 (nearest even).  The prompt's
     * tokens attend over the unrounded keys/values of the prompt (a prefill computes them in
     * one pass); every generated token attends over the rounded cache, its own entry
     * included. */
    int kv_bf16;
} orc_lm_cfg;
/* Weight pointers; layer tensors are stacked [n_layer][...].  Matrices are [out][in].
 * GPT-2: wte[V][d], wpe[ctx][d], ln1_g/b, w_qkv[3d][d], b_qkv[3d], w_o[d][d], b_o[d],
 *        ln2_g/b, w_fc[F][d], b_fc[F], w_proj[d][F], b_proj[d], lnf_g/b.  head = wte.
 * LLaMA: wte[V][d], attn_norm[d], w_qkv[3d][d], w_o[d][d], ffn_norm[d], w_gate[F][d],
 *        w_up[F][d], w_down[d][F], norm_f[d], w_head[V][d]. */
typedef struct {
    const float *wte, *wpe, *ln1_g, *ln1_b, *w_qkv, *b_qkv, *w_o, *b_o, *ln2_g, *ln2_b;
    const float *w_fc, *b_fc, *w_proj, *b_proj, *w_gate, *w_up, *w_down;
    const float *lnf_g, *lnf_b, *w_head;
} orc_lm_weights;
/* greedy generation with a KV cache for B independent sequences.
 * prompt[B][P]; writes out_ids[B][steps]; if logits != NULL writes the logits of every
 * generated step [steps][B][V].  Teacher forcing: if force_ids != NULL the token fed at
 * step s is force_ids[b*steps+s] instead of the argmax (argmax still reported). */
void orc_lm_generate(const orc_lm_cfg *cfg, const orc_lm_weights *w, int B, int P,
                     const int32_t *prompt, int steps, const int32_t *force_ids,
                     int32_t *out_ids, float *logits, int nthreads);
/* one full forward of T tokens (no cache), returning logits of the last position
 * per sequence -- the recompute form the KV-cache path must equal. */
void orc_lm_last_logits(const orc_lm_cfg *cfg, const orc_lm_weights *w, int B, int T,
                        const int32_t *ids, float *logits, int nthreads);
int orc_argmax(const float *x, int n);

#ifdef __cplusplus
}
#endif
#endif
