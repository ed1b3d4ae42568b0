// ref_driver.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Builds the jasmine reference itself (its headers are included by path from the
// reference checkout, nothing is copied) into oracle/_ref/libjasref.so, with plain
// C entry points so tests can (a) pin the C restatement in oracle.c against the real
// reference and (b) write the golden fixtures under tests/golden/, and bench.py can
// time the reference CPU path as its cpu_baseline ("kind": "reference").
//
// Weights are injected through jasmine's own initialiser hook: init_matrix<I>(m)
// dispatches to init_t<I>::cal (mat_init_t.hpp:10-18,113-118), and every net's
// init_weight<I>() visits its matrices in a fixed order (mat_net_t.hpp:51-56,
// mat_mha_t.hpp:141-147,384-392, mat_transformer_kernel_t.hpp:166-176,340-352).
// fixture_init_t fills each visited matrix row-major from a caller buffer.
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>

#include "mat_t.hpp"
#include "mat_express_t.hpp"
#include "mat_view_t.hpp"
#include "mat_net_t.hpp"
#include "mat_init_t.hpp"
#include "mat_mha_t.hpp"
#include "mat_transformer_kernel_t.hpp"
#include "mat_RoPE_t.hpp"
#include "mat_transformer_t.hpp"

struct fixture_init_t;
static const float *g_fixture = nullptr;
static size_t g_fixture_pos = 0;

template <>
struct init_t<fixture_init_t>
{
    template <typename mat_type>
    requires is_matrix<mat_type>
    static void cal(mat_type &m)
    {
        for (int i = 0; i < m.row_num(); ++i)
            for (int j = 0; j < m.col_num(); ++j)
                m(i, j) = g_fixture[g_fixture_pos++];
    }
};

// tanh as a jasmine unary node, built on the reference's own CRTP base
// (mat_express_t.hpp:360-436) exactly like mat_exp_t (:439-469).
template <typename val_type>
class ref_tanh_t : public mat_express_1_param_stable_t<val_type, ref_tanh_t>
{
public:
    using base_type = mat_express_1_param_stable_t<val_type, ref_tanh_t>;
    using ele_type = typename val_type::ele_type;
    using val_base_type = typename base_type::val_base_type;
    ref_tanh_t(val_type const &v) : base_type(v) {}
    auto work(val_base_type i) const { return std::tanh(i); }
    static std::string type_name() { return "ref_tanh_t"; }
};
template <typename val_type>
auto ref_tanh(val_type const &v) { return ref_tanh_t<val_type>(v); }

static mat_t<float> to_mat(const float *p, int R, int C)
{
    mat_t<float> m(R, C);
    for (int i = 0; i < R; ++i)
        for (int j = 0; j < C; ++j) m(i, j) = p[(long)i * C + j];
    return m;
}

template <typename M>
static void from_mat(const M &m, float *out)
{
    int R = m.row_num(), C = m.col_num();
    for (int i = 0; i < R; ++i)
        for (int j = 0; j < C; ++j) out[(long)i * C + j] = static_cast<float>(m(i, j));
}

template <typename T>
using upd_t = sgd_t<T>;

struct hash_init_t;
template <>
struct init_t<hash_init_t>
{
    template <typename mat_type>
    requires is_matrix<mat_type>
    static void cal(mat_type &m)
    {
        for (int i = 0; i < m.row_num(); ++i)
            for (int j = 0; j < m.col_num(); ++j)
                m(i, j) = (float)(((uint32_t)(i * 2654435761u) ^ (uint32_t)(j * 40503u)) % 2001 - 1000) * 2e-5f;
    }
};

static void rms_rows(mat_t<float> &h, const mat_t<float> &x, int d)
{
    double ss = 0;
    for (int i = 0; i < d; ++i) ss += (double)x(i, 0) * x(i, 0);
    const float r = (float)(1.0 / std::sqrt(ss / d + 1e-6));
    for (int i = 0; i < d; ++i) h(i, 0) = x(i, 0) * r;
}

extern "C" {

// mat_t::dot -> mat_dot_t clone (mat_express_t.hpp:730-776)
void ref_gemm(int M, int N, int K, const float *A, const float *B, float *C)
{
    auto a = to_mat(A, M, K), b = to_mat(B, K, N);
    mat_t<float> c = a.dot(b).clone();
    from_mat(c, C);
}

// A.t().dot(B) through mat_view_t transposition (mat_view_t.hpp:97-102)
void ref_gemm_tn(int M, int N, int K, const float *A /*[K,M]*/, const float *B, float *C)
{
    auto a = to_mat(A, K, M), b = to_mat(B, K, N);
    mat_t<float> c = a.t().dot(b).clone();
    from_mat(c, C);
}

void ref_cfg2_expr(const float *A, const float *B, const float *C, float *D, int R, int Cc)
{
    auto a = to_mat(A, R, Cc), b = to_mat(B, R, Cc), c = to_mat(C, R, Cc);
    mat_t<float> d = (a * b + 0.5 * c - ref_tanh(a)).clone();
    from_mat(d, D);
}

// generic small expressions used to pin the ew interpreter: id selects the tree.
void ref_expr(int id, const float *A, int ar, int ac, const float *B, int br, int bc,
              float *out, int *out_r, int *out_c)
{
    auto a = to_mat(A, ar, ac), b = to_mat(B, br, bc);
    mat_t<float> r;
    switch (id) {
    case 0: r = (a + b).clone(); break;
    case 1: r = (a - b * 2).clone(); break;
    case 2: r = (a * b / (b + 3.0)).clone(); break;
    case 3: r = exp(a - b).clone(); break;
    case 4: r = sigmoid(a * b).clone(); break;
    case 5: r = ((a > b) * a + (a < b) * b).clone(); break;
    case 6: r = ((a + b - a) * b / a).clone(); break;
    case 7: r = (a - 1.5f).clone(); break;
    case 8: r = (2 - a).clone(); break;
    case 9: r = (a.t() * 0.25 + b).clone(); break;
    default: throw std::invalid_argument("ref_expr id");
    }
    *out_r = r.row_num();
    *out_c = r.col_num();
    if (out) from_mat(r, out);
}

void ref_hsoftmax(const float *X, int R, int C, float *Y)
{
    auto x = to_mat(X, R, C);
    mat_t<float> y = hsoftmax(x);
    from_mat(y, Y);
}

void ref_softmax_global(const float *X, int R, int C, float *Y)
{
    auto x = to_mat(X, R, C);
    mat_t<float> y = softmax(x).clone();
    from_mat(y, Y);
}

void ref_reductions(const float *X, int R, int C, float *hs, float *vs, float *hm,
                    float *vmn, float *hmn, float *scalars /*sum,max,mean*/)
{
    auto x = to_mat(X, R, C);
    from_mat(hsum(x), hs);
    from_mat(vsum(x), vs);
    from_mat(hmax(x), hm);
    from_mat(vmean(x), vmn);
    from_mat(hmean(x), hmn);
    scalars[0] = sum(x);
    scalars[1] = max(x);
    scalars[2] = mean(x);
}

void ref_linear(const float *W, const float *b, const float *X, int out, int in, int T, float *Y)
{
    weight_net_t<mat_t<float>, upd_t> net(in, out);
    std::vector<float> buf((size_t)out * in + out);
    memcpy(buf.data(), W, sizeof(float) * out * in);
    memcpy(buf.data() + (size_t)out * in, b, sizeof(float) * out);
    g_fixture = buf.data(); g_fixture_pos = 0;
    net.init_weight<fixture_init_t>();
    auto x = to_mat(X, in, T);
    from_mat(net.forward(x), Y);
}

void ref_relu(const float *X, int R, int C, float *Y)
{
    relu_net_t<mat_t<float>> n;
    from_mat(n.forward(to_mat(X, R, C)), Y);
}

void ref_sigmoid(const float *X, int R, int C, float *Y)
{
    sigmoid_net_t<mat_t<float>> n;
    from_mat(n.forward(to_mat(X, R, C)), Y);
}

void ref_layernorm_cols(const float *X, int R, int C, float *Y)
{
    layer_norm_net_t<mat_t<float>, upd_t> n;
    from_mat(n.forward(to_mat(X, R, C)), Y);
}

// mat_head_gen_t self (Xkv == NULL) or cross attention
void ref_head(const float *Xq, const float *Xkv, int dh, int Tq, int Tk, const float *W, int mask, float *Y)
{
    mat_head_gen_t<mat_t<float>, upd_t> head(dh, mask != 0, Tq);
    g_fixture = W; g_fixture_pos = 0;
    head.init_weight<fixture_init_t>();
    auto xq = to_mat(Xq, dh, Tq);
    if (!Xkv) {
        from_mat(head.forward(xq.view()), Y);
    } else {
        auto xk = to_mat(Xkv, dh, Tk);
        from_mat(head.forward(xq.view(), xk.view()), Y);
    }
}

void ref_mha(const float *Xq, const float *Xkv, int d, int H, int Tq, int Tk, const float *W, int mask, float *Y)
{
    mat_mha_t<mat_t<float>, upd_t> mha(H, d, mask != 0, Tq);
    g_fixture = W; g_fixture_pos = 0;
    mha.init_weight<fixture_init_t>();
    auto xq = to_mat(Xq, d, Tq);
    if (!Xkv) {
        from_mat(mha.forward(xq), Y);
    } else {
        auto xk = to_mat(Xkv, d, Tk);
        from_mat(mha.forward(xq, xk), Y);
    }
}

void ref_rope(const float *X, int d, int T, float *Y)
{
    RoPE_net_t<mat_t<float>> r(d);
    from_mat(r.forward(to_mat(X, d, T)), Y);
}

// transformer_base_t: encoder_forward then forward (mat_transformer_t.hpp:36-44)
void ref_transformer(const float *en, int Te, const float *de, int Td, int d, int H,
                     int n_enc, int n_dec, const float *W, float *Y)
{
    transformer_base_t<mat_t<float>, upd_t> tf(n_enc, n_dec, H, d);
    g_fixture = W; g_fixture_pos = 0;
    tf.init_weight<fixture_init_t>();
    tf.encoder_forward(to_mat(en, d, Te));
    from_mat(tf.forward(to_mat(de, d, Td)), Y);
}

// the decode loop of test_transformer_t::predict (transformer_test.hpp:227-239) without the
// harness's SOS/EOS flag rows: column 0 of the decoder input is given; each step runs
// forward on the prefix view [0, len) and appends the output's last column.  Y receives the
// d x (steps + 1) sequence.
void ref_predict_loop(const float *en, int Te, const float *de0, int d, int H, int n_enc, int n_dec,
                      const float *W, int steps, float *Y)
{
    transformer_base_t<mat_t<float>, upd_t> tf(n_enc, n_dec, H, d);
    g_fixture = W; g_fixture_pos = 0;
    tf.init_weight<fixture_init_t>();
    tf.encoder_forward(to_mat(en, d, Te));
    mat_t<float> seq(d, steps + 1);
    for (int i = 0; i < d; ++i) seq(i, 0) = de0[i];
    int len = 1;
    for (int s = 0; s < steps; ++s) {
        auto cur = seq.view(0, 0, d, len);
        auto out = tf.forward(cur);
        seq.col(len++).assign(out.back_col());
    }
    from_mat(seq, Y);
}

// number of parameters transformer_base_t::init_weight visits (for buffer sizing)
long ref_transformer_nparams(int d, int H, int n_enc, int n_dec)
{
    transformer_base_t<mat_t<float>, upd_t> tf(n_enc, n_dec, H, d);
    static std::vector<float> zeros;
    zeros.assign(1 << 24, 0.0f);
    g_fixture = zeros.data(); g_fixture_pos = 0;
    tf.init_weight<fixture_init_t>();
    return (long)g_fixture_pos;
}

// ---- CPU-baseline timers (seconds per call of the reference code path) ----
// weight_net_t::forward at a real projection shape (mat_net_t.hpp:38-49)
double ref_time_linear(int out, int in, int T, int reps)
{
    weight_net_t<mat_t<float>, upd_t> net(in, out);
    std::vector<float> buf((size_t)out * in + out);
    for (size_t i = 0; i < buf.size(); ++i) buf[i] = (float)((i * 2654435761u) % 1000) * 1e-5f;
    g_fixture = buf.data(); g_fixture_pos = 0;
    net.init_weight<fixture_init_t>();
    mat_t<float> x(in, T);
    for (int i = 0; i < in; ++i)
        for (int j = 0; j < T; ++j) x(i, j) = 0.001f * (float)((i + j) % 7);
    volatile float sink = 0.0f;
    auto t0 = std::chrono::steady_clock::now();
    for (int r = 0; r < reps; ++r) {
        auto y = net.forward(x);
        sink = sink + y(0, 0);
    }
    auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<double>(t1 - t0).count() / reps;
}

// the config-2 fused expression, R x C (mat_express_t.hpp:96-107 clone loop)
double ref_time_cfg2(int R, int C, int reps)
{
    mat_t<float> a(R, C), b(R, C), c(R, C);
    for (int i = 0; i < R; ++i)
        for (int j = 0; j < C; ++j) { a(i, j) = 0.1f * (float)((i + j) % 13); b(i, j) = 0.5f; c(i, j) = 1.0f; }
    volatile double sink = 0;
    auto t0 = std::chrono::steady_clock::now();
    for (int r = 0; r < reps; ++r) {
        mat_t<float> d = (a * b + 0.5 * c - ref_tanh(a)).clone();
        sink = sink + d(0, 0);
    }
    auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<double>(t1 - t0).count() / reps;
}

// hsoftmax at R x C (mat_express_t.hpp:681-694)
double ref_time_hsoftmax(int R, int C, int reps)
{
    mat_t<float> a(R, C);
    for (int i = 0; i < R; ++i)
        for (int j = 0; j < C; ++j) a(i, j) = 0.1f * (float)((i * 7 + j) % 13);
    volatile float sink = 0;
    auto t0 = std::chrono::steady_clock::now();
    for (int r = 0; r < reps; ++r) {
        mat_t<float> y = hsoftmax(a);
        sink = sink + y(0, 0);
    }
    auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<double>(t1 - t0).count() / reps;
}

// one masked mat_head_gen_t forward of T tokens at head dim dh (mat_mha_t.hpp:45-74)
double ref_time_head(int dh, int T, int reps)
{
    mat_head_gen_t<mat_t<float>, upd_t> head(dh, true, T);
    std::vector<float> buf(3 * ((size_t)dh * dh + dh), 0.01f);
    g_fixture = buf.data(); g_fixture_pos = 0;
    head.init_weight<fixture_init_t>();
    mat_t<float> x(dh, T);
    for (int i = 0; i < dh; ++i)
        for (int j = 0; j < T; ++j) x(i, j) = 0.01f * (float)((i + 3 * j) % 11);
    volatile float sink = 0;
    auto t0 = std::chrono::steady_clock::now();
    for (int r = 0; r < reps; ++r) {
        auto y = head.forward(x.view());
        sink = sink + y(0, 0);
    }
    auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<double>(t1 - t0).count() / reps;
}


// ---- one LLaMA-shaped decode step of one sequence, on jasmine's own objects ----
// jasmine has no KV cache, RMSNorm, RoPE or SwiGLU (its decode loop recomputes the prefix,
// transformer_test.hpp:194-242).  The step is timed as jasmine code would compute it with
// a cache held in mat_t: the seven projections through weight_net_t::forward
// (mat_net_t.hpp:38-49), per head S = q^T K / sqrt(d_h) with mat_dot_t and the double
// division (mat_mha_t.hpp:53), hsoftmax (mat_express_t.hpp:681-694) and V P^T
// (mat_mha_t.hpp:71); the O(d) glue (RMSNorm, rotary, SiLU gate, residual adds) as plain
// loops.  Only the time is used.
// seconds for one layer of one sequence's decode step over a T-key cache; *attn_s gets the
// attention part (scores, softmax, weighted sum over all heads)
double ref_time_llama_layer(int d, int H, int F, int T, double *attn_s)
{
    using M = mat_t<float>;
    const int dh = d / H;
    weight_net_t<M, upd_t> wq(d, d), wk(d, d), wv(d, d), wo(d, d), wg(d, F), wu(d, F), wd(F, d);
    // weights and cache keep mat_t's zero initialisation: filling 1.3 G elements through
    // operator() would take longer than the timed step, and x86 fp32 arithmetic time does not
    // depend on the values (no denormals arise from zeros)
    std::vector<M> kc, vc;
    for (int h = 0; h < H; ++h) {
        kc.emplace_back(dh, T);
        vc.emplace_back(dh, T);
    }
    M x(d, 1), hbuf(d, 1), att(d, 1);
    for (int i = 0; i < d; ++i) x(i, 0) = 0.01f * (float)(i % 17);
    volatile float sink = 0;
    auto t0 = std::chrono::steady_clock::now();
    rms_rows(hbuf, x, d);
    M q = wq.forward(hbuf), k = wk.forward(hbuf), v = wv.forward(hbuf);
    for (int i = 0; i < d; i += 2) {  // rotary on q and k (position T)
        const double a = T / std::pow(10000.0, (double)(i % dh) / dh);
        const float c = (float)std::cos(a), s = (float)std::sin(a);
        const float q0 = q(i, 0), q1 = q(i + 1, 0), k0 = k(i, 0), k1 = k(i + 1, 0);
        q(i, 0) = q0 * c - q1 * s; q(i + 1, 0) = q0 * s + q1 * c;
        k(i, 0) = k0 * c - k1 * s; k(i + 1, 0) = k0 * s + k1 * c;
    }
    auto ta = std::chrono::steady_clock::now();
    for (int h = 0; h < H; ++h) {
        M qh = q.view(h * dh, 0, dh, 1);
        auto scores = (qh.t().dot(kc[h]) / sqrt(dh)).clone();
        auto p = hsoftmax(scores);
        auto o = vc[h].dot(p.t()).clone();
        for (int e = 0; e < dh; ++e) att(h * dh + e, 0) = o(e, 0);
    }
    auto tb = std::chrono::steady_clock::now();
    M o = wo.forward(att);
    for (int i = 0; i < d; ++i) x(i, 0) = x(i, 0) + o(i, 0);
    rms_rows(hbuf, x, d);
    M g = wg.forward(hbuf), u = wu.forward(hbuf);
    M ff(F, 1);
    for (int i = 0; i < F; ++i) ff(i, 0) = g(i, 0) / (1.0f + std::exp(-g(i, 0))) * u(i, 0);
    M dn = wd.forward(ff);
    for (int i = 0; i < d; ++i) x(i, 0) = x(i, 0) + dn(i, 0);
    sink = sink + x(0, 0) + (float)k(0, 0) + (float)v(0, 0);
    auto t1 = std::chrono::steady_clock::now();
    if (attn_s) *attn_s = std::chrono::duration<double>(tb - ta).count();
    return std::chrono::duration<double>(t1 - t0).count();
}

// ---- GPT-2-shaped decode step of one sequence, on jasmine's own objects ----
// As ref_time_llama_layer, for the GPT-2 block (config 4): four projections with bias
// through weight_net_t::forward (QKV as three d x d nets, O, FC d -> F, proj F -> d), the same
// per-head attention over a T-key cache, and the O(d) glue (row LayerNorm, GELU, residual
// adds) as plain loops.  Seconds for one layer; *attn_s gets the attention part.
static void ln_rows(mat_t<float> &h, const mat_t<float> &x, int d)
{
    double m = 0, v = 0;
    for (int i = 0; i < d; ++i) m += x(i, 0);
    m /= d;
    for (int i = 0; i < d; ++i) v += (x(i, 0) - m) * (x(i, 0) - m);
    const float r = (float)(1.0 / std::sqrt(v / d + 1e-5));
    for (int i = 0; i < d; ++i) h(i, 0) = (float)(x(i, 0) - m) * r;
}

double ref_time_gpt2_layer(int d, int H, int F, int T, double *attn_s)
{
    using M = mat_t<float>;
    const int dh = d / H;
    weight_net_t<M, upd_t> wq(d, d), wk(d, d), wv(d, d), wo(d, d), wf(d, F), wp(F, d);
    std::vector<M> kc, vc;
    for (int h = 0; h < H; ++h) {
        kc.emplace_back(dh, T);
        vc.emplace_back(dh, T);
    }
    M x(d, 1), hbuf(d, 1), att(d, 1);
    for (int i = 0; i < d; ++i) x(i, 0) = 0.01f * (float)(i % 17);
    volatile float sink = 0;
    auto t0 = std::chrono::steady_clock::now();
    ln_rows(hbuf, x, d);
    M q = wq.forward(hbuf), k = wk.forward(hbuf), v = wv.forward(hbuf);
    auto ta = std::chrono::steady_clock::now();
    for (int h = 0; h < H; ++h) {
        M qh = q.view(h * dh, 0, dh, 1);
        auto scores = (qh.t().dot(kc[h]) / sqrt(dh)).clone();
        auto p = hsoftmax(scores);
        auto o = vc[h].dot(p.t()).clone();
        for (int e = 0; e < dh; ++e) att(h * dh + e, 0) = o(e, 0);
    }
    auto tb = std::chrono::steady_clock::now();
    M o = wo.forward(att);
    for (int i = 0; i < d; ++i) x(i, 0) = x(i, 0) + o(i, 0);
    ln_rows(hbuf, x, d);
    M f = wf.forward(hbuf);
    for (int i = 0; i < F; ++i) {
        const float z = f(i, 0);
        f(i, 0) = 0.5f * z * (1.0f + std::tanh(0.7978845608f * (z + 0.044715f * z * z * z)));
    }
    M pr = wp.forward(f);
    for (int i = 0; i < d; ++i) x(i, 0) = x(i, 0) + pr(i, 0);
    sink = sink + x(0, 0) + (float)k(0, 0) + (float)v(0, 0);
    auto t1 = std::chrono::steady_clock::now();
    if (attn_s) *attn_s = std::chrono::duration<double>(tb - ta).count();
    return std::chrono::duration<double>(t1 - t0).count();
}

// ---- one layer of a T-token prefill slice, on jasmine's own objects ----
// kind 0 (GPT-2 block: QKV, O, FC, proj) or 1 (LLaMA block: QKV, O, gate, up, down), every
// projection through weight_net_t::forward on a [d, T] token matrix (mat_dot_t over the T
// columns), causal attention per head as mat_head_gen_t computes it after its projections
// (scores, mask, hsoftmax, V P^T; mat_mha_t.hpp:53-71); norms and activations are O(d T) and
// left out.  Seconds for the layer; *attn_s gets the attention part, which grows with T^2
// where the projections grow with T.
double ref_time_prefill_layer(int kind, int d, int H, int F, int T, double *attn_s)
{
    using M = mat_t<float>;
    const int dh = d / H;
    weight_net_t<M, upd_t> wq(d, d), wk(d, d), wv(d, d), wo(d, d), w1(d, F), w2(F, d), w3(d, F);
    M x(d, T);
    init_matrix<hash_init_t>(x);
    volatile float sink = 0;
    auto t0 = std::chrono::steady_clock::now();
    M q = wq.forward(x), k = wk.forward(x), v = wv.forward(x);
    auto ta = std::chrono::steady_clock::now();
    M att(d, T);
    for (int h = 0; h < H; ++h) {
        M qh = q.view(h * dh, 0, dh, T), kh = k.view(h * dh, 0, dh, T), vh = v.view(h * dh, 0, dh, T);
        auto scores = (qh.t().dot(kh) / sqrt(dh)).clone();
        for (int i = 0; i < T; ++i)
            for (int j = i + 1; j < T; ++j) scores(i, j) = -std::numeric_limits<float>::infinity();
        auto p = hsoftmax(scores);
        auto o = vh.dot(p.t()).clone();
        for (int e = 0; e < dh; ++e)
            for (int t = 0; t < T; ++t) att(h * dh + e, t) = o(e, t);
    }
    auto tb = std::chrono::steady_clock::now();
    M o = wo.forward(att);
    M f = w1.forward(o);
    if (kind == 1) {
        M u = w3.forward(o);
        sink = sink + u(0, 0);
    }
    M dn = w2.forward(f);
    sink = sink + dn(0, 0);
    auto t1 = std::chrono::steady_clock::now();
    if (attn_s) *attn_s = std::chrono::duration<double>(tb - ta).count();
    return std::chrono::duration<double>(t1 - t0).count();
}

// one causal attention head of S tokens at head dim dh without its projections (the
// scores, mask, softmax and weighted sum of mat_head_gen_t::forward, mat_mha_t.hpp:53-71)
double ref_time_attention_head(int dh, int S)
{
    using M = mat_t<float>;
    M q(dh, S), k(dh, S), v(dh, S);
    init_matrix<hash_init_t>(q); init_matrix<hash_init_t>(k); init_matrix<hash_init_t>(v);
    volatile float sink = 0;
    auto t0 = std::chrono::steady_clock::now();
    auto scores = (q.t().dot(k) / sqrt(dh)).clone();
    for (int i = 0; i < scores.row_num(); ++i)
        for (int j = i + 1; j < scores.col_num(); ++j) scores(i, j) = -std::numeric_limits<float>::infinity();
    auto p = hsoftmax(scores);
    auto o = v.dot(p.t()).clone();
    sink = sink + o(0, 0);
    auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<double>(t1 - t0).count();
}

} // extern "C"
