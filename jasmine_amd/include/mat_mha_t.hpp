// Attention of jasmine's API (mat_mha_t.hpp:9-453 of the reference) on the MI355X kernels.
//
// mat_head_gen_t keeps jasmine's head semantics: each head owns d_h x d_h projections of
// its own row slice of the input, scores are Q'K / sqrt(d_h) computed as a float GEMM then
// divided in double (the int sqrt makes the node double), the causal mask sets j > i to
// -inf, hsoftmax, then V P'.  Every step is a device kernel (GEMM, elementwise, mask, row
// softmax); only shapes cross to the host.
#ifndef __MAT_MHA_T_HPP__
#define __MAT_MHA_T_HPP__
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

    void step()
    {
        m_q_net.step();
        m_k_net.step();
        m_v_net.step();
    }
};

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

public:
    mat_mha_t(int num_heads = 1, int d_model = 1, bool mask = false, int seq_len = 1)
        : m_output_proj(d_model, d_model), m_num_heads(num_heads), m_d_model(d_model),
          m_d_head(num_heads ? d_model / num_heads : 0)
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
        m_heads.resize(num_heads);
        for (int i = 0; i < num_heads; ++i) m_heads[i].set_param(m_d_head, mask, seq_len);
        m_output_proj.reinit(std::vector<int>{d_model, d_model});
    }

    mat_t<val_type> forward(const input_type &input)
    {
        if (input.row_num() != m_d_model) throw std::runtime_error("Input row dimension must match d_model");
        auto splits = vsplit(input, m_num_heads);
        std::vector<mat_t<val_type>> head_outputs;
        head_outputs.reserve(m_num_heads);
        for (int i = 0; i < m_num_heads; ++i) head_outputs.push_back(m_heads[i].forward(splits[i]));
        return m_output_proj.forward(vconcat(head_outputs));
    }

    mat_t<val_type> forward(const input_type &input, const input_type &encoder_input)
    {
        if (input.row_num() != m_d_model) throw std::runtime_error("Input row dimension must match d_model");
        if (encoder_input.row_num() != m_d_model)
            throw std::runtime_error("Encoder input row dimension must match d_model");
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

    mat_t<val_type> backward(const input_type &) { jas::detail::no_training("mat_mhca_t::backward"); }

    void step() { base_type::step(); }
};

#endif
