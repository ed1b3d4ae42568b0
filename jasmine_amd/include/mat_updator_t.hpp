// Optimiser types of jasmine's API (mat_updator_t.hpp:10-218 of the reference).  Training is
// outside the MI355X inference path: the types exist so nets templated on an updator compile
// and keep their hyper-parameters, but update() throws.
#ifndef __MAT_UPDATOR_T_HPP__
#define __MAT_UPDATOR_T_HPP__
#include <stdexcept>

#include "mat_t.hpp"

namespace jas::detail {
[[noreturn]] inline void no_training(const char *who)
{
    throw std::logic_error(std::string(who) + ": training (backward / update) is not part of the MI355X inference path");
}
} // namespace jas::detail

template <typename val_type>
class sgd_t
{
    val_type m_learning_rate;

public:
    sgd_t(val_type learning_rate = 0.001) : m_learning_rate(learning_rate) {}
    void set(val_type learning_rate = 0.001) { m_learning_rate = learning_rate; }
    void set_lr(val_type lr) { m_learning_rate = lr; }
    val_type lr() const { return m_learning_rate; }
    void update(const mat_t<val_type> &, mat_t<val_type> &) { jas::detail::no_training("sgd_t::update"); }
    void step() {}
};

template <typename val_type>
class adam_t
{
    val_type m_learning_rate, m_beta1, m_beta2, m_epsilon;

public:
    adam_t(val_type learning_rate = 0.001, val_type beta1 = 0.9, double beta2 = 0.999, double epsilon = 1e-8)
        : m_learning_rate(learning_rate), m_beta1(beta1), m_beta2((val_type)beta2), m_epsilon((val_type)epsilon)
    {
    }
    void set(val_type learning_rate = 0.001, val_type beta1 = 0.9, double beta2 = 0.999, double epsilon = 1e-8)
    {
        m_learning_rate = learning_rate, m_beta1 = beta1, m_beta2 = (val_type)beta2, m_epsilon = (val_type)epsilon;
    }
    void set_lr(val_type lr) { m_learning_rate = lr; }
    val_type lr() const { return m_learning_rate; }
    void update(const mat_t<val_type> &, mat_t<val_type> &) { jas::detail::no_training("adam_t::update"); }
    void step() {}
};

template <typename val_type>
class nadam_t : public adam_t<val_type>
{
public:
    using adam_t<val_type>::adam_t;
    void update(const mat_t<val_type> &, mat_t<val_type> &) { jas::detail::no_training("nadam_t::update"); }
};

template <typename val_type, template <typename> class updator_type>
class cache_updator_t
{
    updator_type<val_type> m_updator;

public:
    cache_updator_t(val_type learning_rate = 0.001) : m_updator(learning_rate) {}
    void update(const mat_t<val_type> &, mat_t<val_type> &) { jas::detail::no_training("cache_updator_t::update"); }
    void step() {}
    void set_lr(val_type lr) { m_updator.set_lr(lr); }
    template <typename... upr_arg_types>
    void set(val_type learning_rate, upr_arg_types &&...args)
    {
        m_updator.set(learning_rate, std::forward<upr_arg_types>(args)...);
    }
};

#endif
