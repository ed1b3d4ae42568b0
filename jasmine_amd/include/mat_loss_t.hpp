// Loss nets of jasmine's API (mat_loss_t.hpp:11-58 of the reference): forward passes its
// input through; loss() evaluates on the device.  backward() belongs to training.
#ifndef __MAT_LOSS_T_HPP__
#define __MAT_LOSS_T_HPP__
#include <sstream>
#include <string>

#include "mat_concepts.hpp"
#include "mat_express_t.hpp"
#include "mat_updator_t.hpp"

template <typename input_type>
class mat_loss_t
{
public:
    using val_type = typename input_type::ele_type;
    mat_t<val_type> m_input;
    mat_loss_t() = default;
    mat_t<val_type> forward(const input_type &input)
    {
        m_input = jas::materialize(input);
        return m_input;
    }
};

template <typename input_type>
class mse_loss_t : public mat_loss_t<input_type>
{
public:
    using base_type = mat_loss_t<input_type>;
    using val_type = typename base_type::val_type;
    mse_loss_t() = default;
    mat_t<val_type> backward(const mat_t<val_type> &) const { jas::detail::no_training("mse_loss_t::backward"); }
    // mean squared error against a target (mat_loss_t.hpp:42-45)
    val_type loss(const mat_t<val_type> &target) const { return mean(pow(base_type::m_input - target)); }
    std::string net_type(int const &indent = 0) const { return print_indent(indent) + "mse_loss_t"; }
    template <typename init_type>
    void init_weight()
    {
    }
    void step() {}
};

#endif
