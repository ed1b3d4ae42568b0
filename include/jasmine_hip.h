/*
 * jasmine_hip.h -- C ABI of libjasmine_hip.so, the MI355X (gfx950) implementation of
 * jasmine's transformer inference hot path.
 *
 * The reference (a header-only C++20 CPU library) has no FFI of its own: its boundary is
 * the template API.  These entry points are what that API's evaluation points lower to;
 * each declaration names the reference code it replaces (file:line into the jasmine
 * sources).  The C++20 headers under jasmine_amd/include/ (mat_t.hpp, mat_express_t.hpp,
 * mat_net_t.hpp, mat_mha_t.hpp, ...) are the only intended direct callers besides the
 * test/bench bindings.
 *
 * Conventions
 *  - plain pointers and sizes; every pointer argument named d_* is device memory;
 *  - the caller owns every buffer;
 *  - every call is asynchronous on `stream` (a hipStream_t; NULL = the library stream);
 *  - every call returns a jas_status; jas_last_error() gives the message.  The C++
 *    wrapper maps JAS_ERR_INVALID to std::invalid_argument, JAS_ERR_RANGE to
 *    std::out_of_range and everything else to std::runtime_error, the exception types the
 *    reference throws (mat_express_t.hpp:711, mat_mha_t.hpp:240, mat_RoPE_t.hpp:57).
 */
#ifndef JASMINE_HIP_H
#define JASMINE_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    JAS_OK = 0,
    JAS_ERR_INVALID = 1, /* shape / argument mismatch  -> std::invalid_argument */
    JAS_ERR_RUNTIME = 2, /* state error                 -> std::runtime_error    */
    JAS_ERR_HIP = 3,     /* HIP runtime failure                                  */
    JAS_ERR_OOM = 4,     /* device allocation failed                             */
    JAS_ERR_RANGE = 5    /* index / capacity overflow   -> std::out_of_range     */
} jas_status;

typedef void *jas_stream_t;

typedef enum { JAS_F32 = 0, JAS_F64 = 1, JAS_I32 = 2, JAS_BF16 = 3 } jas_dtype;

/* ------------------------------------------------------------------ runtime */
/* Device selection and library stream creation.  Storage behind mat_t<T>
 * (mat_t.hpp:53-69 new[]/memset, :30-42 delete[]). */
jas_status jas_init(int device);
const char *jas_last_error(void);
const char *jas_version(void);
jas_stream_t jas_default_stream(void);
/* Frees the library's scratch buffer for `stream` (NULL: the library stream), which
 * multi-pass kernels (whole-matrix reductions, global softmax, prefill key splits) grow
 * per stream and otherwise keep until the process ends.  Waits for the stream's queued work
 * first.  Call it before destroying a short-lived stream that ran such kernels (never after:
 * a destroyed handle is not a stream); the next such kernel on that stream allocates again.
 * No reference counterpart (jasmine has no streams). */
jas_status jas_stream_release_scratch(jas_stream_t stream);
jas_status jas_malloc(void **d_ptr, size_t bytes);          /* mat_t.hpp:67 new[] */
jas_status jas_free(void *d_ptr);                            /* mat_t.hpp:39 delete[] */
/* Stream-ordered block cache behind the C++ headers' mat_t storage (jasmine allocates and
 * frees per matrix, mat_t.hpp:67 / :39; a device free would synchronise the GPU each time).
 * A released block is reused by the next allocation of its rounded size at once, so the
 * memory may only be used by work on the library stream (NULL stream), as the headers do.
 * jas_pool_trim synchronises that stream and returns every cached block to the device
 * (cached_before may be NULL). */
jas_status jas_pool_alloc(void **d_ptr, size_t bytes);
jas_status jas_pool_free(void *d_ptr);
jas_status jas_pool_trim(size_t *cached_before);
jas_status jas_memset(void *d_ptr, int value, size_t bytes, jas_stream_t stream); /* mat_t.hpp:68 memset */
jas_status jas_memcpy_h2d(void *d_dst, const void *src, size_t bytes, jas_stream_t stream);
jas_status jas_memcpy_d2h(void *dst, const void *d_src, size_t bytes, jas_stream_t stream);
jas_status jas_memcpy_d2d(void *d_dst, const void *d_src, size_t bytes, jas_stream_t stream);
jas_status jas_synchronize(jas_stream_t stream);

/* ------------------------------------------------------------------ L1 expressions */
/* A leaf of an expression tree: a mat_t, or a mat_view_t of one.  Element (i, j) of the
 * leaf is read exactly as jasmine reads it:
 *   view (mat_view_t.hpp:28-38):  (a, b) = transposed ? (j + coff, i + roff) : (i + roff, j + coff)
 *   matrix (mat_t.hpp:312-320):    a %= rows; b %= cols;
 *                                  addr = row_first ? a * cols + b : b * rows + a
 * which also gives jasmine's modulo broadcasting of smaller operands. */
typedef struct {
    const void *d_data;
    int32_t dtype;       /* jas_dtype of the stored elements */
    int32_t rows, cols;  /* dims of the underlying matrix (the modulo bases) */
    int32_t row_first;   /* storage order of the underlying matrix (mat_t.hpp:27) */
    int32_t roff, coff;  /* view offsets (0 for a plain mat_t) */
    int32_t transposed;  /* view transposition flag (mat_view_t.hpp:19) */
    int32_t vrows, vcols;/* logical dims of the leaf as seen by the expression */
} jas_leaf;

/* Postfix instructions.  Each instruction's `dtype` is the C++ ele_type of that node
 * (std::common_type promotion, mat_express_t.hpp:41-44); its result is rounded to that
 * type before a parent consumes it, as the typed work(lval_base_type, rval_base_type)
 * parameters do in jasmine. */
typedef enum {
    JAS_OP_LEAF = 0,   /* push leaf[arg]                                            */
    JAS_OP_CONST = 1,  /* push imm (a scalar operand, stored as 1x1 mat_t<T>)        */
    JAS_OP_ADD = 2,    /* mat_add_t  mat_express_t.hpp:188-223                        */
    JAS_OP_SUB = 3,    /* mat_sub_t  :253-286                                         */
    JAS_OP_MUL = 4,    /* mat_mul_t  :288-321                                         */
    JAS_OP_DIV = 5,    /* mat_div_t  :323-358                                         */
    JAS_OP_GT = 6,     /* mat_greater_t :119-151 (bool result in node dtype)          */
    JAS_OP_LT = 7,     /* mat_less_t :153-186                                         */
    JAS_OP_EXP = 8,    /* mat_exp_t :439-469 (exp in the operand's type)              */
    JAS_OP_SIGMOID = 9,/* mat_sigmoid_t :479-509 (1.0/(1.0+exp(-x)), exp in operand type) */
    JAS_OP_TANH = 10,  /* new node: tanh in operand type                              */
    JAS_OP_GELU = 11,  /* new node: 0.5x(1+tanh(sqrt(2/pi)(x+0.044715x^3)))           */
    JAS_OP_SILU = 12,  /* new node: x/(1+exp(-x))                                     */
    JAS_OP_SQRT = 13,  /* sqrt(mat) :804-813                                           */
    JAS_OP_POW = 14,   /* pow(mat, p) :587-596 (std::pow(x, double p))                */
    JAS_OP_NEG = 15    /* unary minus                                                  */
} jas_ew_op;

/* `arg`: leaf index for JAS_OP_LEAF; for binary ops bit 0 set means the right operand
 * was pushed first (Sethi-Ullman order keeps the stack within JAS_EW_MAX_STACK). */
typedef struct {
    int32_t op;
    int32_t dtype;
    int32_t arg;
    int32_t pad;
    double imm;
} jas_ew_ins;

#define JAS_EW_MAX_INS 48
#define JAS_EW_MAX_LEAVES 8
#define JAS_EW_MAX_STACK 4

/* Materialise an expression tree: mat_express_2_param_stable_t::clone / operator mat_t
 * (mat_express_t.hpp:96-112, 416-432).  Output is a dense row-major [rows, cols] matrix
 * of out_dtype (one fused kernel, one HBM pass over the leaves). */
jas_status jas_ew_eval(const jas_ew_ins *prog, int n_ins, const jas_leaf *leaves, int n_leaves,
                       void *d_out, int32_t out_dtype, int rows, int cols, jas_stream_t stream);

/* How jas_ew_eval runs a program (no counterpart in the reference; a tuning switch):
 * 0 = always the interpreter kernel, 1 = always a kernel specialised to the program
 * (compiled once per program shape with hipRTC, cached for the process), 2 = specialise
 * outputs of at least 2^20 elements (default).  Returns the previous mode; other values
 * only query it.  Both paths give identical results. */
int jas_ew_jit_mode(int mode);

/* Reductions over a leaf (mat_express_t.hpp:511-628).  op: 0 sum, 1 max, 2 mean.
 * axis: 0 = per row (hsum/hmax/hmean -> [rows,1]), 1 = per column (vsum/vmean -> [1,cols]),
 * 2 = whole matrix (sum/max/mean -> one value).  Accumulation in out_dtype. */
jas_status jas_reduce(const jas_leaf *in, int op, int axis, void *d_out, int32_t out_dtype,
                      jas_stream_t stream);

/* mat_view_t::assign (mat_view_t.hpp:53-63): write the dense row-major [rows, cols] matrix
 * src (dtype src_dtype) through the view/broadcast mapping of `dst` (element (i, j) of the
 * view, i < rows, j < cols), converting to dst's dtype.  Where jasmine's modulo mapping
 * sends several (i, j) to one element, one of them wins (not necessarily the last). */
jas_status jas_leaf_assign(const void *d_src, int32_t src_dtype, int rows, int cols, const jas_leaf *dst,
                           jas_stream_t stream);

/* ------------------------------------------------------------------ L2 row ops */
/* All row ops act on `n_vec` vectors of length `len`; element e of vector v is read from
 * x[v * x_vstride + e * estride] and written to y[v * y_vstride + e * estride] (row-wise:
 * vstride=len, estride=1; column-wise on a row-major [len, n_vec] matrix: vstride=1,
 * estride=n_vec). */

/* hsoftmax (mat_express_t.hpp:681-694) / hsoftmax_net_t::forward (mat_net_t.hpp:273-279):
 * y = exp(x - max) / sum, one HBM read + one write per vector. */
jas_status jas_softmax(const float *d_x, float *d_y, int n_vec, int len, long x_vstride, long y_vstride,
                       long estride, jas_stream_t stream);
/* The causal mask of mat_head_gen_t::forward (mat_mha_t.hpp:58-67): S[i][j] = value for
 * j > i on a row-major [rows, cols] matrix with leading dimension ld. */
jas_status jas_causal_mask(float *d_S, int rows, int cols, long ld, float value, jas_stream_t stream);
jas_status jas_causal_mask_f64(double *d_S, int rows, int cols, long ld, double value, jas_stream_t stream);
/* whole-matrix softmax mat_softmax_t (mat_express_t.hpp:630-679), dense n floats */
jas_status jas_softmax_global(const float *d_x, float *d_y, long n, jas_stream_t stream);
/* LayerNorm: y = (x - mean) / sqrt(var + eps) * g[e] + b[e]  (population variance).
 * eps = 0 with column layout is jasmine's layer_norm_net_t::forward (mat_net_t.hpp:209-225).
 * g / b may be NULL (1 / 0). */
jas_status jas_layernorm(const float *d_x, float *d_y, int n_vec, int len, long x_vstride, long y_vstride,
                         long estride, float eps, const float *d_g, const float *d_b, jas_stream_t stream);
/* RMSNorm (new): y = x / sqrt(mean(x^2) + eps) * g[e] */
jas_status jas_rmsnorm(const float *d_x, float *d_y, int n_vec, int len, long x_vstride, long y_vstride,
                       long estride, float eps, const float *d_g, jas_stream_t stream);

/* ------------------------------------------------------------------ GEMM */
typedef enum {
    JAS_ACT_NONE = 0,
    JAS_ACT_RELU = 1,    /* relu_net_t (x>0)*x, mat_net_t.hpp:146-153 */
    JAS_ACT_GELU = 2,    /* GPT-2 tanh GELU */
    JAS_ACT_SILU = 3,
    JAS_ACT_SIGMOID = 4  /* sigmoid_net_t, mat_net_t.hpp:101-106 */
} jas_act;

/* C(m, n) = act( sum_k A(m, k) B(k, n) + bias ) (+ C(m, n) if accumulate)
 *   A(m,k) = A[m*as0 + k*as1], B(k,n) = B[k*bs0 + n*bs1], C(m,n) = C[m*cs0 + n*cs1]
 * bias_mode: 0 none, 1 bias[m] (weight_net_t bias broadcast over tokens, mat_net_t.hpp:41),
 *            2 bias[n].
 * Replaces mat_dot_t (mat_express_t.hpp:696-784) and weight_net_t::forward
 * (mat_net_t.hpp:38-49).  fp32 MFMA (v_mfma_f32_16x16x4_f32), fp32 accumulate.
 * `batch` independent problems at element offsets *_bstride (0 = shared operand). */
jas_status jas_gemm(int M, int N, int K,
                    const float *d_A, long as0, long as1,
                    const float *d_B, long bs0, long bs1,
                    float *d_C, long cs0, long cs1,
                    const float *d_bias, int bias_mode, int act, int accumulate,
                    int batch, long a_bstride, long b_bstride, long c_bstride, long bias_bstride,
                    jas_stream_t stream);

/* C(m, n) = act(sum_k A(m, k) B(k, n) + bias) + R(m, n), R(m, n) = R[m*rs0 + n*rs1]: a
 * residual block's last product with the skip connection in its epilogue -- jasmine's
 * residual_net_t::forward (mat_net_t.hpp:326-329) computes f(x) + x with f ending in
 * weight_net_t::forward (mat_net_t.hpp:38-49), optionally followed by relu_net_t /
 * sigmoid_net_t (the encoder-decoder FFN), or in mat_mha_t's output projection; every step
 * is formed in the same order and precision.  One problem (no batch); R must not overlap C. */
jas_status jas_gemm_residual(int M, int N, int K,
                             const float *d_A, long as0, long as1,
                             const float *d_B, long bs0, long bs1,
                             float *d_C, long cs0, long cs1,
                             const float *d_bias, int bias_mode, int act,
                             const float *d_R, long rs0, long rs1, jas_stream_t stream);

/* Same contract in fp64 (mat_dot_t on mat_t<double>), on the fp64 matrix cores
 * (v_mfma_f64_16x16x4_f64); no activation or accumulate, bias_mode 0/1/2 as above. */
jas_status jas_gemm_f64(int M, int N, int K,
                        const double *d_A, long as0, long as1,
                        const double *d_B, long bs0, long bs1,
                        double *d_C, long cs0, long cs1,
                        const double *d_bias, int bias_mode, jas_stream_t stream);

/* ------------------------------------------------------------------ attention */
/* Causal / full flash attention forward, token-major Q[B,H,Sq,D], K,V[B,H,Sk,D] -> O.
 * Replaces the materialised S = Q'K / sqrt(d) -> mask -> hsoftmax -> V P' sequence of
 * mat_head_gen_t::forward (mat_mha_t.hpp:45-74) for dense heads.  Causal aligns the last
 * query with the last key.  dtype JAS_F32 or JAS_BF16 (bf16 inputs, fp32 accumulate).
 * D in {32, 64, 128}.  Strides (elements) select the [B,H,S,D] layout of each tensor:
 * x(b,h,s,:) = x[b*sb + h*sh + s*ss]. */
jas_status jas_attn_prefill(const void *d_Q, const void *d_K, const void *d_V, void *d_O,
                            int B, int H, int Sq, int Sk, int D,
                            long q_sb, long q_sh, long q_ss, long k_sb, long k_sh, long k_ss,
                            long o_sb, long o_sh, long o_ss,
                            float scale, int causal, int dtype, jas_stream_t stream);
/* One-query-per-(b,h) decode step over a KV cache (flash-decoding: split over the keys,
 * log-sum-exp merge by the last split of each (b,h) to finish, in the same launch).
 * q[B,H,D], cache K/V[(b,h)] rows of D at k_sb/k_sh strides, seqlens[B] = number of valid
 * keys per sequence (device int32).  Equivalent to the last column of a full recompute
 * (transformer_test.hpp:231-238 recomputes the prefix).  d_work must hold
 * jas_attn_decode_workspace(B, H, D, max_len) bytes of split partials (no initialisation;
 * calls that share it must not overlap).  The splits' arrival counters are the library's,
 * one zeroed array per stream (jas_stream_release_scratch frees it). */
size_t jas_attn_decode_workspace(int B, int H, int D, int max_len);
jas_status jas_attn_decode(const float *d_q, const float *d_K, const float *d_V, float *d_O,
                           const int32_t *d_seqlens, int B, int H, int D, int max_len,
                           long k_sb, long k_sh, float scale, void *d_work, jas_stream_t stream);

/* jas_attn_decode without a workspace and without any device allocation: no counterpart in
 * the reference (jasmine allocates per matrix).  It is for callers that cannot allocate --
 * code under HIP graph capture, serving loops, harnesses that forbid hipMalloc.  The split
 * partials go to a static device array of jas_attn_decode_scratch_max() bytes (8 MiB) per
 * GPU, with a second static array of 65536 split-arrival counters, held until the process
 * ends; shapes whose partials (jas_attn_decode_workspace(B, H, D, max_len)) exceed the
 * scratch, or that split over more than 65536 (b, h) pairs, are rejected with JAS_ERR_INVALID
 * (the split count stays within two to four workgroups per CU, so on a 256-CU MI355X every shape's
 * partials stay below 1 MiB and none is rejected).
 * Every call on one GPU shares that array: calls that overlap on one GPU (two streams, or
 * two host threads) race.  Results are identical to jas_attn_decode's. */
#define JAS_DECODE_SCRATCH_BYTES ((size_t)8 << 20)
size_t jas_attn_decode_scratch_max(void);
jas_status jas_attn_decode_noalloc(const float *d_q, const float *d_K, const float *d_V, float *d_O,
                                   const int32_t *d_seqlens, int B, int H, int D, int max_len,
                                   long k_sb, long k_sh, float scale, jas_stream_t stream);

/* ------------------------------------------------------------------ RoPE, embeddings, argmax */
/* jasmine RoPE_net_t::forward (mat_RoPE_t.hpp:166-188) with mat_RoPE_t::init angles
 * (mat_RoPE_t.hpp:107-131); x, y row-major [d, T] feature-major. */
jas_status jas_rope_jasmine(const float *d_x, float *d_y, int d, int T, jas_stream_t stream);
jas_status jas_rope_jasmine_f64(const double *d_x, double *d_y, int d, int T, jas_stream_t stream);
/* LLaMA rotary on interleaved pairs, in place: x[(n * nh + h) * hstride ...], n tokens with
 * positions pos[n] (device int32), nh heads of dh each, token stride tstride elements. */
jas_status jas_rope_llama(float *d_x, const int32_t *d_pos, int n, int nh, int dh, long tstride,
                          float theta, jas_stream_t stream);
/* out[n][d] = wte[ids[n]] (+ wpe[pos[n]] if d_wpe) -- token embedding gather (new) */
jas_status jas_embed(const float *d_wte, const float *d_wpe, const int32_t *d_ids, const int32_t *d_pos,
                     float *d_out, int n, int d, jas_stream_t stream);
/* argmax over each of n rows of length V (first maximum wins) */
jas_status jas_argmax(const float *d_x, int n, int V, long ld, int32_t *d_out, jas_stream_t stream);
/* Seeded N(mean, std) fill, same counter-based generator as the host side. */
jas_status jas_fill_normal(float *d_x, size_t n, uint64_t seed, uint64_t stream_id, float mean, float std,
                           jas_stream_t stream);
/* Bandwidth calibration, no counterpart in the reference: a grid-stride streaming read of
 * `bytes` (16-byte aligned, a multiple of 16) by `workgroups` 256-thread workgroups with 4 or
 * 8 16-byte loads in flight per thread, nontemporal or plain.  d_sink (4 bytes) is written
 * only in the unlikely case that the folded data equal a fixed constant.  bench.py uses it
 * as the achievable-read ceiling next to the HBM-bound kernels. */
jas_status jas_hbm_read_probe(const void *d_buf, size_t bytes, int workgroups, int loads_in_flight, int nontemporal,
                              unsigned *d_sink, jas_stream_t stream);

/* ------------------------------------------------------------------ decoder LM runner */
/* Decoder-only language model (GPT-2 / LLaMA shapes).  The reference has no token
 * model (its decode loop is test_transformer_t::predict, transformer_test.hpp:194-242,
 * which recomputes the whole prefix each step); this runner keeps jasmine's decode
 * semantics (each step's output = last column of a full recompute) with a KV cache. */
typedef struct {
    int32_t kind;      /* 0 GPT-2 (pre-LN, GELU, learned positions, tied head), 1 LLaMA */
    int32_t n_layer, d_model, n_head, d_ff, vocab, max_ctx, max_batch;
    float eps, rope_theta;
    /* Storage precision (0 = fp32, the reference's arithmetic; 1 = bf16, round to nearest
     * even).  weight_bf16: the projection matrices and the LM head (GPT-2: the tied
     * embedding) are stored as bf16 and widened to fp32 on load; norms, biases and
     * embeddings stay fp32, every product accumulates in fp32.  kv_bf16: the KV cache holds
     * bf16 keys/values; a prefill attends over the fp32 keys/values it has just computed
     * and stores them rounded, every later step attends over the rounded cache. */
    int32_t weight_bf16, kv_bf16;
} jas_lm_config;

typedef struct jas_lm jas_lm;

jas_status jas_lm_create(const jas_lm_config *cfg, jas_lm **out);
jas_status jas_lm_destroy(jas_lm *lm);
/* Fill every weight N(0, std) from `seed` (norm gains 1, biases 0). */
jas_status jas_lm_init_random(jas_lm *lm, uint64_t seed, float std);
/* Weight tensors by name ("wte", "wpe", "ln1_g", "ln1_b", "w_qkv", "b_qkv", "w_o", "b_o",
 * "ln2_g", "ln2_b", "w_fc", "b_fc", "w_proj", "b_proj", "w_gate", "w_up", "w_down", "lnf_g",
 * "lnf_b", "w_head"); a tensor is `layers` stacked [rows][cols] matrices ([out][in] for
 * projections).  Host copies use that logical row-major order whatever the device layout
 * (projection matrices are stored in the MFMA-native packed layout).  weight_shape reports
 * 0/0/0 for a tensor the model kind lacks.  Stands in for jasmine's init_weight<I>()
 * traversal hook (mat_init_t.hpp:113-118) as the way to load trained weights. */
jas_status jas_lm_weight_shape(jas_lm *lm, const char *name, int *layers, int *rows, int *cols);
jas_status jas_lm_get_weight(jas_lm *lm, const char *name, float *h_dst, size_t count);
jas_status jas_lm_set_weight(jas_lm *lm, const char *name, const float *h_src, size_t count);
/* Prefill B prompts of length P (host int32 ids [B][P]) and return the greedy next ids
 * (host [B]); logits of the last position go to h_logits [B][V] if not NULL. */
jas_status jas_lm_prefill(jas_lm *lm, int B, int P, const int32_t *h_ids, int32_t *h_next, float *h_logits);
/* One decode step for all B sequences: feeds `h_ids` (host [B], or NULL to feed the
 * previous step's argmax kept on the device), appends to the KV cache, returns argmax
 * ids (host [B], NULL = keep on device) and optionally logits [B][V]. */
jas_status jas_lm_decode(jas_lm *lm, const int32_t *h_ids, int32_t *h_next, float *h_logits);
/* Run `steps` greedy decode steps without host round trips; ids out [steps][B] (host). */
jas_status jas_lm_generate(jas_lm *lm, int steps, int32_t *h_ids);
/* jas_lm_generate replays one decode step captured as a HIP graph (default, enable = 1);
 * enable = 0 launches the same kernels eagerly each step (identical results).  No
 * counterpart in the reference: an execution-mode switch, e.g. for tools that cannot
 * follow graph launches. */
jas_status jas_lm_use_graph(jas_lm *lm, int enable);
/* Current sequence length (tokens in the KV cache). */
int jas_lm_position(jas_lm *lm);
/* Key splits of the runner's decode attention at batch B (1 = one pass, no merge;
 * above 1 = split over the cache plus the log-sum-exp merge by the last split to finish; 0 = bad argument).  A query
 * for tests and tuning: no reference counterpart (jasmine has no KV cache). */
int jas_lm_attn_splits(jas_lm *lm, int B);
/* The decode GEMM geometry the runner's step launches for one projection ("w_qkv", "w_o",
 * "w_fc", "w_proj", "w_gate_up", "w_down", "w_head" / "wte"): geo[0] 16-row weight tiles per
 * workgroup (gate/up pairs count two), geo[1] waves per workgroup, geo[2] K chunks in
 * flight per wave, geo[3] K splits (1 = unsplit).  A query for tests and tuning, so a test
 * can show which kernel variant it covered; no reference counterpart. */
jas_status jas_lm_proj_geometry(jas_lm *lm, const char *name, int *geo);
/* One of the runner's stored projections applied to B <= 16 token vectors with the decode
 * step's own weight-streaming GEMM (same kernel variant and geometry): d_y[B][M] = W . x for
 * d_x[B][K] (token-major, device).  Names: "w_qkv", "w_o", "w_fc", "w_proj", "w_down",
 * "w_head" / "wte" (layer ignored) and "w_gate_up" (d_y[B][d_ff] = silu(W_gate x) * (W_up x)).
 * No bias, no activation otherwise.  Runs on `stream` (NULL: the library stream) after
 * draining the runner's stream, whose decode buffers it reuses; before returning it makes the
 * runner's stream wait (on the device) for the projection's last launch, so runner calls may
 * follow without a host synchronisation.  Not thread-safe against a concurrent runner call
 * from another host thread.  No reference counterpart: weight_net_t::forward (mat_net_t.hpp:38-49) on the
 * runner's packed weights, for callers that reuse a layer and for per-kernel measurement. */
jas_status jas_lm_project(jas_lm *lm, const char *name, int layer, int B, const float *d_x, float *d_y,
                          jas_stream_t stream);
jas_stream_t jas_lm_stream(jas_lm *lm);
/* Per-kernel-class GPU time (ms) accumulated with HIP events around every launch on the
 * runner's stream since the last reset; classes: 0 weight GEMM (decode), 1 attention decode,
 * 2 other. enable=0 turns event recording off. */
jas_status jas_lm_profile(jas_lm *lm, int enable, double *ms_by_class, long *launches_by_class);

/* Weight files (safetensors container: 8-byte little-endian header length, JSON header,
 * raw little-endian data).  The reference has no weight file format; its nets take weights
 * only through the init_weight<I>() traversal (mat_init_t.hpp:113-118, mat_net_t.hpp:51-56).
 * Tensors carry the jas_lm_set_weight names, shape [layers, rows, cols] (2-D [rows, cols] is
 * read as one layer) and logical row-major data, F32 or BF16; "__metadata__" holds the
 * config as strings (format = "jasmine_amd.lm").
 * save:  writes every weight (BF16 where the model stores bf16, else F32), atomically
 *        (a temporary file renamed over path).
 * load:  the file must hold exactly this model's tensors with their shapes ("wpe" may have
 *        more positions than max_ctx: its prefix is used); F32 data rounds to bf16 where
 *        the model stores bf16, BF16 data widens exactly to fp32.  The file streams through
 *        pinned staging buffers and is packed on the device; on error the model's weights
 *        are partly overwritten.
 * read_config: the config saved in the file's metadata (host only, no device call). */
jas_status jas_lm_save(jas_lm *lm, const char *path);
jas_status jas_lm_load(jas_lm *lm, const char *path);
jas_status jas_lm_read_config(const char *path, jas_lm_config *cfg);

#ifdef __cplusplus
}
#endif
#endif
