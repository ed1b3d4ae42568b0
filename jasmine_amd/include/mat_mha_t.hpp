// Attention of jasmine's API (mat_mha_t.hpp:9-453 of the reference) on the MI355X kernels.
//
// mat_head_gen_t keeps jasmine's head semantics: each head owns d_h x d_h projections of
// its own row slice of the input, scores are Q'K / sqrt(d_h) computed as a float GEMM then
// divided in double (the int sqrt makes the node double), the causal mask sets j > i to
// -inf, hsoftmax, then V P'.  Every step is a device kernel (GEMM, elementwise, mask, row
// softmax); only shapes cross to the host.
#ifndef __MAT_MHA_T_HPP__
#define __MAT_MHA_T_HPP__
#include <array>
#include <cmath>
#include <limits>
#include <vector>

#include "mat_express_t.hpp"
#include "mat_net_t.hpp"
#include "mat_t.hpp"
#include "mat_view_t.hpp"

namespace jas {
template <typename T>
void causal_mask(mat_t<T> &s)
{
    if (s.is_scalar()) return;  // a single position masks nothing
    const T ninf = -std::numeric_limits<T>::infinity();
    if constexpr (std::is_same_v<T, float>)
        check(jas_causal_mask(s.device_data_mut(), s.row_num(), s.col_num(), s.col_num(), ninf, nullptr));
    else if constexpr (std::is_same_v<T, double>)
        check(jas_causal_mask_f64(s.device_data_mut(), s.row_num(), s.col_num(), s.col_num(), ninf, nullptr));
    else
        for (int i = 0; i < s.row_num(); ++i)
            for (int j = i + 1; j < s.col_num(); ++j) s(i, j) = ninf;
}
} // namespace jas

template <typename input_type, template <typename> class updator_type>
class mat_head_gen_t
{
public:
    using val_type = typename input_type::ele_type;
    using ele_type = typename input_type::ele_type;

private:
    using ffn_type = weight_net_t<input_type, updator_type>;
    using softmax_type = hsoftmax_net_t<input_type>;

    ffn_type m_q_net;
    ffn_type m_k_net;
    ffn_type m_v_net;
    softmax_type m_softmax;
    mat_t<val_type> m_q, m_k, m_v;
    bool m_mask;

    mat_t<val_type> attend(bool mask)
    {
        // Q'K / sqrt(d_h): float GEMM, double division (mat_mha_t.hpp:53)
        auto attn_scores = (m_q.t().dot(m_k) / std::sqrt(m_q.row_num())).clone();
        mat_t<val_type> s(attn_scores);
        if (mask) jas::causal_mask(s);
        auto attn_weights = m_softmax.forward(s);
        return m_v.dot(attn_weights.t()).clone();
    }

public:
    mat_head_gen_t(int const &d_model = 1, bool const &mask = false, int const &seq_len = 1)
        : m_q_net(d_model, d_model), m_k_net(d_model, d_model), m_v_net(d_model, d_model), m_q(d_model, seq_len),
          m_k(d_model, seq_len), m_v(d_model, seq_len), m_mask(mask)
    {
    }

    void set_param(int const &d_model, bool const &mask = false, int const &seq_len = 1)
    {
        m_q_net.reinit(std::vector<int>{d_model, d_model});
        m_k_net.reinit(std::vector<int>{d_model, d_model});
        m_v_net.reinit(std::vector<int>{d_model, d_model});
        m_q.reshape(d_model, seq_len);
        m_k.reshape(d_model, seq_len);
        m_v.reshape(d_model, seq_len);
        m_mask = mask;
    }

    // self attention over the head's rows (mat_mha_t.hpp:45-74)
    template <typename mat_type>
    requires std::is_same_v<std::decay_t<mat_type>, mat_t<val_type>>
    mat_t<val_type> forward(const mat_view_t<mat_type> &input)
    {
        m_q = m_q_net.forward(input);
        m_k = m_k_net.forward(input);
        m_v = m_v_net.forward(input);
        return attend(m_mask);
    }

    // cross attention: queries from the decoder rows, keys/values from the encoder rows
    // (mat_mha_t.hpp:76-90)
    template <typename mat_type>
    requires std::is_same_v<std::decay_t<mat_type>, mat_t<val_type>>
    mat_t<val_type> forward(const mat_view_t<mat_type> &decoder_input, const mat_view_t<mat_type> &encoder_input)
    {
        m_q = m_q_net.forward(decoder_input);
        m_k = m_k_net.forward(encoder_input);
        m_v = m_v_net.forward(encoder_input);
        return attend(false);
    }

    template <typename... args_t>
    mat_t<val_type> backward(args_t &&...)
    {
        jas::detail::no_training("mat_head_gen_t::backward");
    }

    template <typename... upr_arg_types>
    void set_updator(upr_arg_types &&...args)
    {
        m_q_net.set_updator(args...);
        m_k_net.set_updator(args...);
        m_v_net.set_updator(args...);
    }

    template <typename init_type>
    void init_weight()
    {
        m_q_net.template init_weight<init_type>();
        m_k_net.template init_weight<init_type>();
        m_v_net.template init_weight<init_type>();
    }

    std::string net_type(int const &indent = 0) const { return print_indent(indent) + "mat_head_gen_t"; }

    // the head's projections (read by the fused all-heads path of mat_mha_t)
    ffn_type &q_net() { return m_q_net; }
    ffn_type &k_net() { return m_k_net; }
    ffn_type &v_net() { return m_v_net; }

    void step()
    {
        m_q_net.step();
        m_k_net.step();
        m_v_net.step();
    }
};

namespace jas {
// Whether mat_mha_t may run all heads through the fused path (below); the per-head path
// computes the same attention with the score matrix materialised.
inline bool &fused_heads_enabled()
{
    static bool on = true;
    return on;
}

namespace detail {
// Device scratch of the fused path.  A copied net starts with an empty cache.
struct mha_scratch {
    device_buffer w;      // [3][H][d_h][d_h] projection weights, then [3][H][d_h] biases
    device_buffer qkv;    // self: [T][3][H][d_h]; cross: queries [T_q][H][d_h]
    device_buffer kv;     // cross: encoder keys / values [T_k][2][H][d_h]
    device_buffer o;      // attention output [T_q][H][d_h]
    std::vector<uint64_t> w_stamps;
    uint64_t kv_stamp = 0;  // stamp of the encoder output the cached keys / values belong to
    int kv_T = 0;
    mha_scratch() = default;
    mha_scratch(const mha_scratch &) {}
    mha_scratch &operator=(const mha_scratch &)
    {
        w_stamps.clear();
        kv_stamp = 0;
        return *this;
    }
    mha_scratch(mha_scratch &&) noexcept = default;
    mha_scratch &operator=(mha_scratch &&) noexcept = default;
};
} // namespace detail
} // namespace jas

// stack matrices by rows (mat_mha_t.hpp:163-196): device-to-device block copies
template <typename val_type>
mat_t<val_type> vconcat(const std::vector<mat_t<val_type>> &mats)
{
    if (mats.empty()) throw std::runtime_error("Cannot concatenate empty vector");
    const int cols = mats[0].col_num();
    int total_rows = 0;
    for (const auto &m : mats) {
        if (m.col_num() != cols) throw std::runtime_error("All matrices must have the same number of columns");
        total_rows += m.row_num();
    }
    mat_t<val_type> result(total_rows, cols, typename mat_t<val_type>::device_uninit_tag{});
    if (result.is_scalar()) return mats[0];
    int row_offset = 0;
    for (const auto &m : mats) {
        auto block = result.view(row_offset, 0, m.row_num(), cols);
        block.assign(m);
        row_offset += m.row_num();
    }
    return result;
}

// split rows into num_splits views (mat_mha_t.hpp:198-215)
template <typename mat_type>
std::vector<mat_view_t<mat_type>> vsplit(mat_type &mat, int num_splits)
{
    if (num_splits <= 0 || mat.row_num() % num_splits != 0)
        throw std::runtime_error("Invalid number of splits or row count mismatch");
    const int rows_per_split = mat.row_num() / num_splits;
    std::vector<mat_view_t<mat_type>> views;
    for (int i = 0; i < num_splits; ++i) views.emplace_back(mat, i * rows_per_split, 0, rows_per_split, mat.col_num());
    return views;
}

// multi-head attention over row-split heads plus the output projection (mat_mha_t.hpp:221-408)
template <typename input_type, template <typename> class updator_type>
class mat_mha_t
{
public:
    using val_type = typename input_type::ele_type;

private:
    std::vector<mat_head_gen_t<input_type, updator_type>> m_heads;
    weight_net_t<mat_t<val_type>, updator_type> m_output_proj;
    int m_num_heads;
    int m_d_model;
    int m_d_head;
    bool m_mask = false;
    jas::detail::mha_scratch m_fx;

    // All heads at once for float matrices with d_h in {32, 64, 128}: the per-head Q/K/V
    // projections are one batched GEMM (one problem per head, its three blocks stacked;
    // cross attention: Q alone, and K / V of the encoder output) writing token-major rows,
    // attention is the flash kernel over every head (no score matrix in memory), and the
    // output projection reads the token-major result transposed.  Cross attention keeps
    // the encoder-side keys / values while the encoder output and the weights are unchanged.
    // Same arithmetic as the per-head path up to rounding order (scores scaled in float).
    bool fusable(int Tq) const
    {
        if constexpr (!std::is_same_v<val_type, float>) return false;
        else {
            if (!jas::fused_heads_enabled() || Tq < 1) return false;
            if (m_d_head != 32 && m_d_head != 64 && m_d_head != 128) return false;
            auto &self = const_cast<mat_mha_t &>(*this);
            for (auto &hd : self.m_heads)
                for (auto *n : {&hd.q_net(), &hd.k_net(), &hd.v_net()})
                    if (!n->weight().row_first() || n->weight().row_num() != m_d_head ||
                        n->weight().col_num() != m_d_head || n->bias().row_num() != m_d_head ||
                        n->bias().col_num() != 1)
                        return false;
            auto &wo = self.m_output_proj;
            return wo.weight().row_first() && wo.weight().row_num() == m_d_model &&
                   wo.weight().col_num() == m_d_model && wo.bias().row_num() == m_d_model && wo.bias().col_num() == 1;
        }
    }

    // gather the heads' weights and biases into one block (when any of them changed)
    const float *packed_weights()
    {
        const int H = m_num_heads, dh = m_d_head;
        std::vector<uint64_t> st;
        st.reserve(6 * H);
        for (auto &hd : m_heads)
            for (auto *n : {&hd.q_net(), &hd.k_net(), &hd.v_net()}) {
                st.push_back(n->weight().stamp());
                st.push_back(n->bias().stamp());
            }
        if (st != m_fx.w_stamps) {
            m_fx.w.allocate(sizeof(float) * 3 * H * ((size_t)dh * dh + dh));
            float *w = (float *)m_fx.w.get();
            float *b = w + (size_t)3 * H * dh * dh;
            for (int h = 0; h < H; ++h) {
                const std::array<weight_net_t<input_type, updator_type> *, 3> ns{
                    &m_heads[h].q_net(), &m_heads[h].k_net(), &m_heads[h].v_net()};
                for (int sct = 0; sct < 3; ++sct) {  // per head: q, k, v stacked (3 dh rows)
                    const size_t i = (size_t)h * 3 + sct;
                    jas::check(jas_memcpy_d2d(w + i * dh * dh, ns[sct]->weight().device_data(),
                                              sizeof(float) * dh * dh, nullptr));
                    jas::check(jas_memcpy_d2d(b + i * dh, ns[sct]->bias().device_data(), sizeof(float) * dh, nullptr));
                }
            }
            // device_data() may have uploaded a host mirror: stamps are unchanged by that
            m_fx.w_stamps = std::move(st);
            m_fx.kv_stamp = 0;
        }
        return (const float *)m_fx.w.get();
    }

    // projection `sct` (0 q, 1 k, 2 v) of every head: out(n, h*dh + m) at out[n*ld + h*dh + m]
    void project(int sct, const jas::gemm_operand_t<float> &x, int T, float *out, long ld)
    {
        const int H = m_num_heads, dh = m_d_head;
        const float *w = (const float *)m_fx.w.get();
        const float *b = w + (size_t)3 * H * dh * dh + (size_t)sct * dh;
        jas::check(jas_gemm(dh, T, dh, w + (size_t)sct * dh * dh, dh, 1, x.p, x.s0, x.s1, out, 1, ld, b, 1,
                            JAS_ACT_NONE, 0, H, 3L * dh * dh, (long)dh * x.s0, dh, 3L * dh, nullptr));
    }

    // q, k and v of every head in one batched product (one problem per head, its three
    // d_h x d_h blocks stacked): out(n, h, s, m) at out[n*3d + h*3dh + s*dh + m]
    void project_qkv(const jas::gemm_operand_t<float> &x, int T, float *out)
    {
        const int H = m_num_heads, dh = m_d_head;
        const float *w = (const float *)m_fx.w.get();
        const float *b = w + (size_t)3 * H * dh * dh;
        jas::check(jas_gemm(3 * dh, T, dh, w, dh, 1, x.p, x.s0, x.s1, out, 1, 3L * m_d_model, b, 1, JAS_ACT_NONE, 0,
                            H, 3L * dh * dh, (long)dh * x.s0, 3L * dh, 3L * dh, nullptr));
    }

    mat_t<val_type> fused_forward(const input_type &input, const input_type *encoder_input,
                                  const mat_t<val_type> *residual = nullptr)
    {
        const int d = m_d_model, H = m_num_heads, dh = m_d_head, Tq = input.col_num();
        packed_weights();
        auto xq = jas::gemm_operand<float>(input);
        const float *Q, *K, *V;
        long qs, ks, qh = dh, kh = dh;  // token and head strides
        int Tk;
        if (!encoder_input) {
            Tk = Tq;
            m_fx.qkv.allocate(sizeof(float) * (size_t)Tq * 3 * d);
            float *qkv = (float *)m_fx.qkv.get();
            project_qkv(xq, Tq, qkv);
            Q = qkv, K = qkv + dh, V = qkv + 2 * dh, qs = ks = 3L * d, qh = kh = 3L * dh;
        } else {
            Tk = encoder_input->col_num();
            m_fx.qkv.allocate(sizeof(float) * (size_t)Tq * d);
            float *q = (float *)m_fx.qkv.get();
            project(0, xq, Tq, q, d);
            // matrices carry a content stamp; other input types recompute every call
            uint64_t es = 0;
            if constexpr (requires { encoder_input->stamp(); }) es = encoder_input->stamp();
            if (es == 0 || m_fx.kv_stamp != es || m_fx.kv_T != Tk) {
                auto xe = jas::gemm_operand<float>(*encoder_input);
                m_fx.kv.allocate(sizeof(float) * (size_t)Tk * 2 * d);
                float *kv = (float *)m_fx.kv.get();
                project(1, xe, Tk, kv, 2L * d);
                project(2, xe, Tk, kv + d, 2L * d);
                m_fx.kv_stamp = es;
                m_fx.kv_T = Tk;
            }
            const float *kv = (const float *)m_fx.kv.get();
            Q = q, K = kv, V = kv + d, qs = d, ks = 2L * d;
        }
        m_fx.o.allocate(sizeof(float) * (size_t)Tq * d);
        float *o = (float *)m_fx.o.get();
        const bool causal = !encoder_input && m_mask;
        jas::check(jas_attn_prefill(Q, K, V, o, 1, H, Tq, Tk, dh, (long)Tq * qs, qh, qs, (long)Tk * ks, kh, ks,
                                    (long)Tq * d, dh, d, (float)(1.0 / std::sqrt((double)dh)), causal ? 1 : 0,
                                    JAS_F32, nullptr));
        // y = W_o . concat(heads) + b_o, the concatenation read from the token-major rows
        auto &wo = m_output_proj;
        mat_t<val_type> y(d, Tq, typename mat_t<val_type>::device_uninit_tag{});
        if (residual) {  // residual_net_t's + x in the projection's epilogue
            const long r0 = residual->row_first() ? Tq : 1, r1 = residual->row_first() ? 1 : d;
            jas::check(jas_gemm_residual(d, Tq, d, wo.weight().device_data(), d, 1, o, 1, d, y.device_data_mut(), Tq, 1,
                                         wo.bias().device_data(), 1, JAS_ACT_NONE, residual->device_data(), r0, r1,
                                         nullptr));
            return y;
        }
        jas::check(jas_gemm(d, Tq, d, wo.weight().device_data(), d, 1, o, 1, d, y.device_data_mut(), Tq, 1,
                            wo.bias().device_data(), 1, JAS_ACT_NONE, 0, 1, 0, 0, 0, 0, nullptr));
        return y;
    }

public:
    mat_mha_t(int num_heads = 1, int d_model = 1, bool mask = false, int seq_len = 1)
        : m_output_proj(d_model, d_model), m_num_heads(num_heads), m_d_model(d_model),
          m_d_head(num_heads ? d_model / num_heads : 0), m_mask(mask)
    {
        if (num_heads <= 0 || d_model % num_heads != 0) throw std::runtime_error("d_model must be divisible by num_heads");
        for (int i = 0; i < num_heads; ++i) m_heads.emplace_back(m_d_head, mask, seq_len);
    }

    void set_param(int num_heads, int d_model, bool mask = false, int seq_len = 1)
    {
        if (num_heads <= 0 || d_model % num_heads != 0) throw std::runtime_error("d_model must be divisible by num_heads");
        m_num_heads = num_heads;
        m_d_model = d_model;
        m_d_head = d_model / num_heads;
        m_mask = mask;
        m_heads.resize(num_heads);
        for (int i = 0; i < num_heads; ++i) m_heads[i].set_param(m_d_head, mask, seq_len);
        m_output_proj.reinit(std::vector<int>{d_model, d_model});
    }

    mat_t<val_type> forward(const input_type &input)
    {
        if (input.row_num() != m_d_model) throw std::runtime_error("Input row dimension must match d_model");
        if (fusable(input.col_num())) return fused_forward(input, nullptr);
        auto splits = vsplit(input, m_num_heads);
        std::vector<mat_t<val_type>> head_outputs;
        head_outputs.reserve(m_num_heads);
        for (int i = 0; i < m_num_heads; ++i) head_outputs.push_back(m_heads[i].forward(splits[i]));
        return m_output_proj.forward(vconcat(head_outputs));
    }

    // forward(input) + residual with the residual added in the output projection's epilogue
    // (residual_net_t, mat_net_t.hpp:326-329); false: not fused
    bool forward_residual_into(const input_type &input, const mat_t<val_type> &residual, mat_t<val_type> &y)
    {
        if (!fusable(input.col_num()) || residual.is_scalar() || residual.row_num() != m_d_model ||
            residual.col_num() != input.col_num())
            return false;
        y = fused_forward(input, nullptr, &residual);
        return true;
    }
    bool forward_residual_into(const input_type &input, const input_type &encoder_input,
                               const mat_t<val_type> &residual, mat_t<val_type> &y)
    {
        if (!fusable(input.col_num()) || encoder_input.col_num() < 1 || residual.is_scalar() ||
            residual.row_num() != m_d_model || residual.col_num() != input.col_num())
            return false;
        y = fused_forward(input, &encoder_input, &residual);
        return true;
    }

    mat_t<val_type> forward(const input_type &input, const input_type &encoder_input)
    {
        if (input.row_num() != m_d_model) throw std::runtime_error("Input row dimension must match d_model");
        if (encoder_input.row_num() != m_d_model)
            throw std::runtime_error("Encoder input row dimension must match d_model");
        if (fusable(input.col_num()) && encoder_input.col_num() >= 1) return fused_forward(input, &encoder_input);
        auto splits = vsplit(input, m_num_heads);
        auto enc_splits = vsplit(encoder_input, m_num_heads);
        std::vector<mat_t<val_type>> head_outputs;
        head_outputs.reserve(m_num_heads);
        for (int i = 0; i < m_num_heads; ++i) head_outputs.push_back(m_heads[i].forward(splits[i], enc_splits[i]));
        return m_output_proj.forward(vconcat(head_outputs));
    }

    template <typename... args_t>
    mat_t<val_type> backward(args_t &&...)
    {
        jas::detail::no_training("mat_mha_t::backward");
    }

    template <typename... upr_arg_types>
    void set_updator(upr_arg_types &&...args)
    {
        for (auto &head : m_heads) head.set_updator(args...);
        m_output_proj.set_updator(args...);
    }

    // heads in order, then the output projection (mat_mha_t.hpp:384-392)
    template <typename init_type>
    void init_weight()
    {
        for (auto &head : m_heads) head.template init_weight<init_type>();
        m_output_proj.template init_weight<init_type>();
    }

    std::string net_type(int const &indent = 0) const
    {
        return print_indent(indent) + "MHA(heads:" + std::to_string(m_num_heads) + ", d_model:" +
               std::to_string(m_d_model) + ")";
    }

    void step()
    {
        for (auto &head : m_heads) head.step();
        m_output_proj.step();
    }
};

// cross attention against a stored encoder output (mat_mha_t.hpp:410-453)
template <typename input_type, template <typename> class updator_type>
class mat_mhca_t : public mat_mha_t<input_type, updator_type>
{
public:
    using base_type = mat_mha_t<input_type, updator_type>;
    using val_type = typename input_type::ele_type;

private:
    mat_t<val_type> *m_encoder_output = nullptr;
    mat_t<val_type> *m_encoder_delta = nullptr;

public:
    mat_mhca_t(int num_heads = 1, int d_model = 1, bool mask = false, int seq_len = 1)
        : base_type(num_heads, d_model, mask, seq_len)
    {
    }

    void set_encoder_param(mat_t<val_type> &encoder_output, mat_t<val_type> &encoder_delta)
    {
        m_encoder_output = &encoder_output;
        m_encoder_delta = &encoder_delta;
    }

    mat_t<val_type> forward(const input_type &input)
    {
        if (m_encoder_output == nullptr) throw std::runtime_error("Encoder output not set for cross attention");
        return base_type::forward(input, *m_encoder_output);
    }

    // cross attention: the residual rides in the output projection over the encoder output
    bool forward_residual_into(const input_type &input, const mat_t<val_type> &residual, mat_t<val_type> &y)
    {
        if (m_encoder_output == nullptr) throw std::runtime_error("Encoder output not set for cross attention");
        return base_type::forward_residual_into(input, *m_encoder_output, residual, y);
    }

    mat_t<val_type> backward(const input_type &) { jas::detail::no_training("mat_mhca_t::backward"); }

    void step() { base_type::step(); }
};

#endif
