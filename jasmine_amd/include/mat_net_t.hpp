// Layers and composition of jasmine's API (mat_net_t.hpp:12-508 of the reference), forward
// on the MI355X kernels.  Same net protocol: forward(input) -> mat_t, init_weight<I>(),
// set_updator(args...), step(), net_type(indent), reinit({in, out}) for resizable nets,
// residual / complex composition and complex_net_builder_t.  backward() belongs to
// training and throws.
#ifndef __MAT_NET_T_HPP__
#define __MAT_NET_T_HPP__
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "mat_express_t.hpp"
#include "mat_init_t.hpp"
#include "mat_t.hpp"
#include "mat_updator_t.hpp"

namespace jas {

// Y = W . X + b with b a [out, 1] column broadcast over the tokens (weight_net_t::forward,
// mat_net_t.hpp:38-49): one GEMM with the bias in its epilogue
template <typename T, typename X>
mat_t<T> linear(const mat_t<T> &W, const X &x, const mat_t<T> &b)
{
    const int M = W.row_num(), N = x.col_num(), K = W.col_num();
    if (K != x.row_num()) throw std::invalid_argument("mat_dot_t: inner dimensions do not match for dot product");
    const bool fused = !W.is_scalar() && W.row_first() && !b.is_scalar() && b.row_num() == M && b.col_num() == 1 &&
                       !(M == 1 && N == 1) && (std::is_same_v<T, float> || std::is_same_v<T, double>);
    if (!fused) return materialize(dot(W, x) + b);
    auto xo = gemm_operand<T>(x);
    mat_t<T> y(M, N, typename mat_t<T>::device_uninit_tag{});
    if constexpr (std::is_same_v<T, float>)
        check(jas_gemm(M, N, K, W.device_data(), K, 1, xo.p, xo.s0, xo.s1, y.device_data_mut(), N, 1, b.device_data(),
                       1, JAS_ACT_NONE, 0, 1, 0, 0, 0, 0, nullptr));
    else if constexpr (std::is_same_v<T, double>)
        check(jas_gemm_f64(M, N, K, W.device_data(), K, 1, xo.p, xo.s0, xo.s1, y.device_data_mut(), N, 1,
                           b.device_data(), 1, nullptr));
    return y;
}

// act(W . X + b) + R with the skip connection added in the product's epilogue, for
// residual_net_t over a linear layer (mat_net_t.hpp:326-329): each value is formed in the
// order jasmine forms it (the biased product, then the activation, then + R).  Returns false
// when the operands do not fit (the caller then takes jasmine's separate passes).
template <typename T, typename X>
bool linear_residual(const mat_t<T> &W, const X &x, const mat_t<T> &b, int act, const mat_t<T> &R, mat_t<T> &y)
{
    if constexpr (!std::is_same_v<T, float>) {
        return false;
    } else {
        const int M = W.row_num(), N = x.col_num(), K = W.col_num();
        if (K != x.row_num()) throw std::invalid_argument("mat_dot_t: inner dimensions do not match for dot product");
        const bool ok = !W.is_scalar() && W.row_first() && !b.is_scalar() && b.row_num() == M && b.col_num() == 1 &&
                        !(M == 1 && N == 1) && !R.is_scalar() && R.row_num() == M && R.col_num() == N;
        if (!ok) return false;
        auto xo = gemm_operand<T>(x);
        mat_t<T> out(M, N, typename mat_t<T>::device_uninit_tag{});
        const long r0 = R.row_first() ? N : 1, r1 = R.row_first() ? 1 : M;
        check(jas_gemm_residual(M, N, K, W.device_data(), K, 1, xo.p, xo.s0, xo.s1, out.device_data_mut(), N, 1,
                                b.device_data(), 1, act, R.device_data(), r0, r1, nullptr));
        y = std::move(out);
        return true;
    }
}

// column LayerNorm with population std and eps = 0 (layer_norm_net_t::forward,
// mat_net_t.hpp:209-225), gamma/beta per row
template <typename T, typename X>
mat_t<T> layer_norm_cols(const X &input, const mat_t<T> &gamma, const mat_t<T> &beta)
{
    if constexpr (std::is_same_v<T, float>) {
        auto x = as_dense<float>(input);
        const int R = x->row_num(), C = x->col_num();
        if (R > 1 && !gamma.is_scalar() && !beta.is_scalar()) {
            mat_t<float> y(R, C, mat_t<float>::device_uninit_tag{});
            check(jas_layernorm(x->device_data(), y.device_data_mut(), C, R, 1, 1, C, 0.0f, gamma.device_data(),
                                beta.device_data(), nullptr));
            return y;
        }
    }
    // jasmine's own sequence of passes on the generic kernels
    mat_t<T> m_mean = vmean(input);
    auto delta = input - m_mean;
    mat_t<T> m_std = sqrt(vmean(pow(delta.clone(), 2.0)));
    mat_t<T> m_hx = delta / m_std;
    return (gamma * m_hx + beta).clone();
}

} // namespace jas

template <typename input_type, template <typename> class updator_type>
class weight_net_t
{
public:
    using val_type = typename input_type::ele_type;

private:
    mat_t<val_type> m_weight;
    updator_type<val_type> m_weight_updator;
    mat_t<val_type> m_bias;
    updator_type<val_type> m_bias_updator;

public:
    weight_net_t(int const &input_size = 1, int const &output_size = 1)
        : m_weight(output_size, input_size), m_weight_updator(), m_bias(output_size, 1), m_bias_updator()
    {
    }

    void reinit(std::vector<int> const &container)
    {
        m_weight.reshape(container[1], container[0]);
        m_bias.reshape(container[1], 1);
    }

    mat_t<val_type> forward(const input_type &input) { return jas::linear(m_weight, input, m_bias); }

    // act(forward(input)) + residual as one product (used by residual_net_t); false: not fused
    bool forward_act_residual_into(const input_type &input, int act, const mat_t<val_type> &residual,
                                   mat_t<val_type> &y)
    {
        return jas::linear_residual(m_weight, input, m_bias, act, residual, y);
    }
    bool forward_residual_into(const input_type &input, const mat_t<val_type> &residual, mat_t<val_type> &y)
    {
        return forward_act_residual_into(input, JAS_ACT_NONE, residual, y);
    }

    template <typename init_type>
    void init_weight()
    {
        init_matrix<init_type>(m_weight);
        init_matrix<init_type>(m_bias);
    }

    template <typename... upr_arg_types>
    void set_updator(upr_arg_types &&...args)
    {
        m_weight_updator.set(std::forward<upr_arg_types>(args)...);
        m_bias_updator.set(std::forward<upr_arg_types>(args)...);
    }

    template <typename other_type>
    mat_t<val_type> backward(const other_type &)
    {
        jas::detail::no_training("weight_net_t::backward");
    }

    std::string net_type(int const &indent = 0) const
    {
        std::stringstream ss;
        ss << print_indent(indent) << "weight_net_t:(in:" << m_weight.col_num() << ", out:" << m_weight.row_num()
           << ")";
        return ss.str();
    }

    void step()
    {
        m_weight_updator.step();
        m_bias_updator.step();
    }

    mat_t<val_type> &weight() { return m_weight; }
    mat_t<val_type> &bias() { return m_bias; }
};

template <typename input_type>
class sigmoid_net_t
{
public:
    using val_type = typename input_type::ele_type;
    sigmoid_net_t() = default;
    mat_t<val_type> forward(const input_type &input) { return sigmoid(input).clone(); }
    template <typename other_type>
    auto backward(const other_type &)
    {
        jas::detail::no_training("sigmoid_net_t::backward");
    }
    std::string net_type(int const &indent = 0) const { return print_indent(indent) + "sigmoid_net_t"; }
    template <typename init_type>
    void init_weight()
    {
    }
    void step() {}
};

template <typename input_type>
class relu_net_t
{
public:
    using val_type = typename input_type::ele_type;
    relu_net_t() = default;
    // the product epilogue's activation that computes exactly this forward
    static constexpr int jas_fused_act = JAS_ACT_RELU;
    // (x > 0) * x, so negative inputs give -0 and -inf gives NaN as in mat_net_t.hpp:152
    mat_t<val_type> forward(const input_type &input) { return ((input > 0) * input).clone(); }
    template <typename other_type>
    auto backward(const other_type &)
    {
        jas::detail::no_training("relu_net_t::backward");
    }
    std::string net_type(int const &indent = 0) const { return print_indent(indent) + "relu_net_t"; }
    template <typename init_type>
    void init_weight()
    {
    }
    void step() {}
};

// column-wise LayerNorm (normalises each token column of a [features, tokens] input)
template <typename input_type, template <typename> class updator_type>
class layer_norm_net_t
{
public:
    using val_type = typename input_type::ele_type;

private:
    mat_t<val_type> m_gama;  // per-feature scale, created as 1 on first forward
    updator_type<val_type> m_gama_updator;
    mat_t<val_type> m_beta;  // per-feature shift, created as 0 on first forward
    updator_type<val_type> m_beta_updator;

public:
    layer_norm_net_t() = default;

    template <typename... upr_arg_types>
    void set_updator(upr_arg_types &&...args)
    {
        m_gama_updator.set(std::forward<upr_arg_types>(args)...);
        m_beta_updator.set(std::forward<upr_arg_types>(args)...);
    }

    mat_t<val_type> forward(const input_type &input)
    {
        if (!m_gama.valid()) {  // lazily created gamma = 1, beta = 0 (mat_net_t.hpp:215-223)
            m_gama = mat_t<val_type>(input.row_num(), 1);
            m_beta = mat_t<val_type>(input.row_num(), 1);
            m_gama = val_type(1);
            m_beta = val_type(0);
        }
        return jas::layer_norm_cols(input, m_gama, m_beta);
    }

    template <typename other_type>
    auto backward(const other_type &)
    {
        jas::detail::no_training("layer_norm_net_t::backward");
    }

    std::string net_type(int const &indent = 0) const { return print_indent(indent) + "layer_norm_net_t"; }

    template <typename init_type>
    void init_weight()
    {
        init_matrix<init_type>(m_gama);
        init_matrix<init_type>(m_beta);
    }

    void step()
    {
        m_gama_updator.step();
        m_beta_updator.step();
    }
};

template <typename input_type>
class hsoftmax_net_t
{
public:
    using val_type = typename input_type::ele_type;
    mat_t<val_type> m_output;
    mat_t<val_type> forward(const input_type &input)
    {
        m_output = hsoftmax(input);
        return m_output;
    }
    mat_t<val_type> backward(const mat_t<val_type> &) { jas::detail::no_training("hsoftmax_net_t::backward"); }
    std::string net_type(int const &indent = 0) const { return print_indent(indent) + "hsoftmax_net_t"; }
    template <typename init_type>
    void init_weight()
    {
    }
    void step() {}
};

template <typename base_net_type>
class residual_net_t
{
public:
    using val_type = typename base_net_type::val_type;
    base_net_type m_net;

    residual_net_t() : m_net() {}
    base_net_type &base_net() { return m_net; }
    base_net_type const &base_net() const { return m_net; }

    // f(x) + x (mat_net_t.hpp:326-329); where f ends in a product, the + x rides in that
    // product's epilogue (same values, one launch fewer)
    mat_t<val_type> forward(const mat_t<val_type> &input)
    {
        if constexpr (requires(mat_t<val_type> &y) { m_net.forward_residual_into(input, input, y); }) {
            mat_t<val_type> y;
            if (m_net.forward_residual_into(input, input, y)) return y;
        }
        return m_net.forward(input) + input;
    }

    template <typename other_type>
    auto backward(const other_type &)
    {
        jas::detail::no_training("residual_net_t::backward");
    }

    std::string net_type(int const &indent = 0) const
    {
        return print_indent(indent) + "residual_net_t:\n" + m_net.net_type(indent + 2);
    }

    template <typename init_type>
    void init_weight()
    {
        m_net.template init_weight<init_type>();
    }

    template <size_t... nums>
    decltype(auto) get()
    {
        return m_net.template get<nums...>();
    }
    template <size_t... nums>
    decltype(auto) get() const
    {
        return m_net.template get<nums...>();
    }

    template <typename... upr_arg_types>
    void set_updator(upr_arg_types &&...args)
    {
        if constexpr (is_updatable_net<base_net_type>) m_net.set_updator(std::forward<upr_arg_types>(args)...);
    }

    void step() { m_net.step(); }
};

// a tuple of nets applied in order (mat_net_t.hpp:366-488)
template <typename... net_types>
class complex_net_t
{
    std::tuple<net_types...> m_nets;

    template <typename container_type, size_t N, size_t I>
    void reinit_from(container_type const &container)
    {
        using mbr = std::tuple_element_t<N, std::tuple<net_types...>>;
        if constexpr (is_reinitable_net<mbr>) {
            if (I + 1 >= container.size()) throw std::runtime_error("container size does not match net size");
            std::get<N>(m_nets).reinit({container[I], container[I + 1]});
            if constexpr (N + 1 < sizeof...(net_types)) reinit_from<container_type, N + 1, I + 1>(container);
        } else if constexpr (N + 1 < sizeof...(net_types)) {
            reinit_from<container_type, N + 1, I>(container);
        }
    }

public:
    using val_type = typename std::tuple_element_t<0, std::tuple<net_types...>>::val_type;

    template <typename input_type>
    auto forward(const input_type &input)
    {
        return std::apply([&input](auto &&...nets) { return net_forward(input, nets...); }, m_nets);
    }

    // forward(input) + residual with the residual added in the last product's epilogue, when
    // the chain is one linear layer, optionally followed by relu (the encoder-decoder FFN);
    // false: not fused
    template <typename input_type>
    bool forward_residual_into(const input_type &input, const mat_t<val_type> &residual, mat_t<val_type> &y)
    {
        using first_t = std::tuple_element_t<0, std::tuple<net_types...>>;
        if constexpr (!requires(first_t &f, mat_t<val_type> &o) { f.forward_act_residual_into(input, 0, residual, o); }) {
            return false;
        } else if constexpr (sizeof...(net_types) == 1) {
            return std::get<0>(m_nets).forward_act_residual_into(input, JAS_ACT_NONE, residual, y);
        } else if constexpr (sizeof...(net_types) == 2) {
            using second_t = std::tuple_element_t<1, std::tuple<net_types...>>;
            if constexpr (requires { second_t::jas_fused_act; })
                return std::get<0>(m_nets).forward_act_residual_into(input, second_t::jas_fused_act, residual, y);
            else
                return false;
        } else {
            return false;
        }
    }

    template <typename input_type>
    auto backward(const input_type &)
    {
        jas::detail::no_training("complex_net_t::backward");
    }

    constexpr size_t size() { return sizeof...(net_types); }

    // consecutive dimensions {d0, d1, d2, ...} go to the resizable member nets in order
    template <typename container_type>
    void reinit(container_type const &container)
    {
        reinit_from<container_type, 0, 0>(container);
    }

    template <typename... upr_arg_types>
    void set_updator(upr_arg_types &&...args)
    {
        std::apply(
            [&](auto &&...nets) {
                (
                    [&](auto &n) {
                        if constexpr (is_updatable_net<std::decay_t<decltype(n)>>) n.set_updator(args...);
                    }(nets),
                    ...);
            },
            m_nets);
    }

    template <typename init_type>
    void init_weight()
    {
        std::apply([](auto &&...nets) { (nets.template init_weight<init_type>(), ...); }, m_nets);
    }

    void step()
    {
        std::apply([](auto &&...nets) { (nets.step(), ...); }, m_nets);
    }

    std::string net_type(int const &indent = 0) const
    {
        std::stringstream ss;
        ss << print_indent(indent) << "complex_net_t = [";
        std::apply([&ss, indent](auto &&...nets) { ((ss << std::endl << nets.net_type(indent + 2)), ...); }, m_nets);
        ss << std::endl << print_indent(indent) << "]";
        return ss.str();
    }

    auto back() { return std::get<sizeof...(net_types) - 1>(m_nets); }

    template <size_t N, size_t... nums>
    decltype(auto) get()
    {
        if constexpr (sizeof...(nums) == 0) return (std::get<N>(m_nets));
        else return std::get<N>(m_nets).template get<nums...>();
    }
    template <size_t N, size_t... nums>
    decltype(auto) get() const
    {
        if constexpr (sizeof...(nums) == 0) return (std::get<N>(m_nets));
        else return std::get<N>(m_nets).template get<nums...>();
    }
};

// type-level builder of complex_net_t (mat_net_t.hpp:494-508)
template <typename val_type, typename... net_types>
struct complex_net_builder_t {
    template <template <typename, template <typename> class> class cur_net_tpl, template <typename> class updator_tpl>
    using push_back_updatable = complex_net_builder_t<val_type, net_types..., cur_net_tpl<mat_t<val_type>, updator_tpl>>;

    template <template <typename> class cur_net_tpl>
    using push_back_staticnet = complex_net_builder_t<val_type, net_types..., cur_net_tpl<mat_t<val_type>>>;

    template <typename new_net_type>
    using push_back_impl = complex_net_builder_t<val_type, net_types..., new_net_type>;

    using type = complex_net_t<net_types...>;
};

#include "mat_loss_t.hpp"

#endif
