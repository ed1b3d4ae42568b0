// Weight initialisers of jasmine's API (mat_init_t.hpp:8-118 of the reference): init_t<I>
// specialisations filled through mat_t's element access (host mirror, uploaded on the
// next device use), init_matrix<I>(m) as the hook every net's init_weight<I>() calls.
#ifndef __MAT_INIT_T_HPP__
#define __MAT_INIT_T_HPP__
#include <cmath>
#include <random>

#include "mat_concepts.hpp"
#include "mat_t.hpp"

inline std::default_random_engine g_random_engine;

template <typename init_type>
struct init_t {
    template <typename mat_type>
    requires is_matrix<mat_type>
    static void cal(mat_type &)
    {
    }
};

namespace jas::detail {
template <typename mat_type, typename dist_type>
void fill_dist(mat_type &m, dist_type dist)
{
    for (int i = 0; i < m.row_num(); ++i)
        for (int j = 0; j < m.col_num(); ++j) m(i, j) = dist(g_random_engine);
}
} // namespace jas::detail

template <>
struct init_t<class zeros_t> {
    template <typename mat_type>
    requires is_matrix<mat_type>
    static void cal(mat_type &m)
    {
        for (int i = 0; i < m.row_num(); ++i)
            for (int j = 0; j < m.col_num(); ++j) m(i, j) = 0;
    }
};

template <>
struct init_t<class xavier_gaussian_t> {
    template <typename mat_type>
    requires is_matrix<mat_type>
    static void cal(mat_type &m)
    {
        jas::detail::fill_dist(m, std::normal_distribution<double>(0.0, std::sqrt(2.0 / (m.row_num() + m.col_num()))));
    }
};

template <>
struct init_t<class xavier_uniform_t> {
    template <typename mat_type>
    requires is_matrix<mat_type>
    static void cal(mat_type &m)
    {
        const double a = std::sqrt(6.0 / (m.row_num() + m.col_num()));
        jas::detail::fill_dist(m, std::uniform_real_distribution<double>(-a, a));
    }
};

template <>
struct init_t<class he_gaussian_t> {
    template <typename mat_type>
    requires is_matrix<mat_type>
    static void cal(mat_type &m)
    {
        jas::detail::fill_dist(m, std::normal_distribution<double>(0.0, std::sqrt(2.0 / m.col_num())));
    }
};

template <>
struct init_t<class he_uniform_t> {
    template <typename mat_type>
    requires is_matrix<mat_type>
    static void cal(mat_type &m)
    {
        const double a = std::sqrt(6.0 / m.col_num());
        jas::detail::fill_dist(m, std::uniform_real_distribution<double>(-a, a));
    }
};

template <typename init_type, typename mat_type, typename... args_types>
requires is_matrix<mat_type>
void init_matrix(mat_type &m, args_types &&...args)
{
    init_t<init_type>::cal(m, std::forward<args_types>(args)...);
}

#endif
