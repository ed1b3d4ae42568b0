// Rotary position embedding of jasmine's API (mat_RoPE_t.hpp:7-230 of the reference).
// mat_RoPE_t keeps the host-side cos/sin cache and forward_unite() views for code that
// inspects rotation blocks; RoPE_net_t::forward runs the rotation as one device kernel with
// the same angle formula (jas_rope_jasmine).
#ifndef __MAT_ROPE_HPP__
#define __MAT_ROPE_HPP__
#include <cmath>
#include <sstream>

#include "mat_express_t.hpp"
#include "mat_view_t.hpp"

// growable cache matrix (mat_RoPE_t.hpp:7-73)
template <typename val_type>
class mat_cache_t
{
    mat_t<val_type> m_cache;
    int m_cache_rows = 0, m_cache_cols = 0;
    static constexpr int EXPAND_SIZE = 1024;

    void expand_cache(int rows, int cols)
    {
        if (rows > m_cache.row_num() || cols > m_cache.col_num()) {
            const int nr = rows > m_cache.row_num() ? std::max(rows, m_cache.row_num() + EXPAND_SIZE) : m_cache.row_num();
            const int nc = cols > m_cache.col_num() ? std::max(cols, m_cache.col_num() + EXPAND_SIZE) : m_cache.col_num();
            mat_t<val_type> grown(nr, nc);
            for (int i = 0; i < m_cache.row_num(); ++i)
                for (int j = 0; j < m_cache.col_num(); ++j) grown(i, j) = m_cache(i, j);
            m_cache = std::move(grown);
        }
    }

public:
    mat_cache_t() : m_cache(EXPAND_SIZE, EXPAND_SIZE) {}

    val_type &operator()(int row, int col)
    {
        if (row >= m_cache_rows || col >= m_cache_cols) {
            expand_cache(row + 1, col + 1);
            m_cache_rows = std::max(m_cache_rows, row + 1);
            m_cache_cols = std::max(m_cache_cols, col + 1);
        }
        return m_cache(row, col);
    }

    const val_type &operator()(int row, int col) const
    {
        if (row >= m_cache_rows || col >= m_cache_cols) throw std::out_of_range("Cache access out of range");
        return m_cache(row, col);
    }

    mat_view_t<mat_t<val_type>> range(int row, int col, int rows, int cols)
    {
        if (row + rows > m_cache_rows || col + cols > m_cache_cols) {
            expand_cache(row + rows, col + cols);
            m_cache_rows = std::max(m_cache_rows, row + rows);
            m_cache_cols = std::max(m_cache_cols, col + cols);
        }
        return m_cache.view(row, col, rows, cols);
    }
};

template <typename val_type>
class mat_RoPE_t
{
    mat_cache_t<val_type> m_cache;
    int m_enable_rows = 0, m_enable_cols = 0;
    int m_d;

public:
    mat_RoPE_t(int const &d) : m_d(d) {}

    void set_d(int const &d)
    {
        m_d = d;
        m_enable_rows = m_enable_cols = 0;
    }

    val_type get_d() const { return m_d; }

    // cache entry (i, j): angle = j / 10000^((i/2) / d) in val_type; cos where i and j have
    // the same parity, -sin at (even, odd), sin at (odd, even) (mat_RoPE_t.hpp:99-134)
    void init(int const &row_beg, int const &rows, int const &col_beg, int const &cols)
    {
        for (int i = 0; i < row_beg + rows; ++i)
            for (int j = 0; j < col_beg + cols; ++j) {
                if (i < m_enable_rows && j < m_enable_cols) continue;
                val_type angle = j / std::pow(10000.0, (i / 2) / static_cast<val_type>(m_d));
                if ((i % 2) == (j % 2)) m_cache(i, j) = std::cos(angle);
                else if (i % 2 == 0) m_cache(i, j) = -std::sin(angle);
                else m_cache(i, j) = std::sin(angle);
            }
        m_enable_rows = row_beg + rows;
        m_enable_cols = col_beg + cols;
    }

    mat_view_t<mat_t<val_type>> range(int row_beg, int row_num, int col_beg, int col_num)
    {
        if (row_beg + row_num >= m_enable_rows || col_beg + col_num >= m_enable_cols)
            init(row_beg, row_num, col_beg, col_num);
        return m_cache.range(row_beg, col_beg, row_num, col_num);
    }

    // the 2x2 rotation block of pair i at position m
    mat_view_t<mat_t<val_type>> forward_unite(int const &i, int const &m) { return range(i * 2, 2, m * 2, 2); }
};

template <typename input_type>
class RoPE_net_t
{
    using val_type = typename input_type::ele_type;
    mat_RoPE_t<val_type> m_rope;

public:
    RoPE_net_t(int const &d_model) : m_rope(d_model) {}

    void set_param(int const &d_model) { m_rope.set_d(d_model); }

    // y[2i..2i+1, m] = block(i, m) . x[2i..2i+1, m] for every token column (mat_RoPE_t.hpp:166-188)
    mat_t<val_type> forward(input_type const &x)
    {
        const int T = x.col_num(), d = x.row_num();
        if (d != (int)m_rope.get_d()) throw std::runtime_error("Input dimension does not match RoPE dimension");
        static_assert(std::is_same_v<val_type, float> || std::is_same_v<val_type, double>,
                      "RoPE runs in float or double");
        auto in = jas::as_dense<val_type>(x);
        mat_t<val_type> ret(d, T, typename mat_t<val_type>::device_uninit_tag{});
        if (ret.is_scalar()) return mat_t<val_type>(val_type{});  // d = 1: no pair, zero output
        if constexpr (std::is_same_v<val_type, float>)
            jas::check(jas_rope_jasmine(in->device_data(), ret.device_data_mut(), d, T, nullptr));
        else
            jas::check(jas_rope_jasmine_f64(in->device_data(), ret.device_data_mut(), d, T, nullptr));
        return ret;
    }

    mat_t<val_type> backward(const mat_t<val_type> &) { jas::detail::no_training("RoPE_net_t::backward"); }

    template <typename>
    void init_weight()
    {
    }
    void step() {}

    std::string net_type(int const &indent = 0) const
    {
        std::stringstream ss;
        ss << print_indent(indent) << "RoPE_net_t:(d_model:" << m_rope.get_d() << ")";
        return ss.str();
    }
};

#endif
