// Printing and net-folding helpers of jasmine's API (mat_utility.hpp:17-100 of the
// reference): operator<< for anything with to_string(), operator>> / net_forward folds that
// thread an input through nets, and print_indent for net_type() dumps.
#ifndef __MAT_UTILITY_HPP__
#define __MAT_UTILITY_HPP__
#include <cmath>
#include <ostream>
#include <string>
#include <tuple>
#include <utility>

#include "mat_concepts.hpp"

template <typename val_type>
requires is_serializable<val_type>
std::ostream &operator<<(std::ostream &os, const val_type &m)
{
    return os << m.to_string();
}

// input >> net == net.forward(input)
template <typename net_type, typename input_type>
requires is_forwardable<net_type, input_type>
auto operator>>(input_type const &input, net_type &net)
{
    return net.forward(input);
}

template <typename input_type, typename... net_types>
auto net_forward(input_type const &input, net_types &&...nets)
{
    return (input >> ... >> nets);
}

template <typename net_type, typename input_type>
requires is_backwardable<net_type, input_type>
auto operator<<(net_type &net, input_type const &input)
{
    return net.backward(input);
}

template <typename... net_type, typename input_type>
auto net_backward(input_type const &input, net_type &&...nets)
{
    return (nets << ... << input);
}

inline std::string print_indent(int const indent)
{
    return std::string(2 * (indent > 0 ? indent : 0), ' ');
}

#endif
