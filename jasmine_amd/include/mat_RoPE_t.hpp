// Rotary position embedding of jasmine's API (mat_RoPE_t.hpp:7-230 of the reference).
// mat_RoPE_t evaluates rotation blocks on the host for code that inspects them
// (forward_unite); RoPE_net_t::forward runs the rotation as one device kernel with the same
// angle formula (jas_rope_jasmine).
#ifndef __MAT_ROPE_HPP__
#define __MAT_ROPE_HPP__
#include <cmath>
#include <sstream>

#include "mat_express_t.hpp"
#include "mat_view_t.hpp"

#include <array>
#include <map>

// Host-side rotation blocks of jasmine's RoPE (mat_RoPE_t.hpp:76-150 of the reference).
// Only inspection code uses them: RoPE_net_t::forward computes every angle on the device.
// Each distinct block request (row_beg, rows, col_beg, cols) is evaluated once from the
// closed form into a matrix of exactly that size and kept for the object's lifetime, so the
// views returned stay valid; a changed d drops every block.
template <typename val_type>
class mat_RoPE_t
{
    using key_t = std::array<int, 4>;
    std::map<key_t, mat_t<val_type>> m_blocks;  // node-based: stored matrices never move
    int m_d;

public:
    mat_RoPE_t(int const &d) : m_d(d) {}

    void set_d(int const &d)
    {
        m_d = d;
        m_blocks.clear();
    }

    val_type get_d() const { return m_d; }

    // Entry (r, c) of jasmine's rotation table (mat_RoPE_t.hpp:113-131): with
    // a = c / 10000^((r/2) / d) evaluated in val_type, cos(a) where r and c have the same
    // parity, -sin(a) at (even r, odd c) and sin(a) at (odd r, even c).
    val_type entry(int r, int c) const
    {
        const val_type a = c / std::pow(10000.0, (r / 2) / static_cast<val_type>(m_d));
        if ((r & 1) == (c & 1)) return std::cos(a);
        return (r & 1) ? std::sin(a) : -std::sin(a);
    }

    // view of rows [row_beg, row_beg + row_num) x columns [col_beg, col_beg + col_num)
    mat_view_t<mat_t<val_type>> range(int row_beg, int row_num, int col_beg, int col_num)
    {
        if (row_beg < 0 || col_beg < 0 || row_num <= 0 || col_num <= 0)
            throw std::out_of_range("mat_RoPE_t::range: empty or negative block");
        auto found = m_blocks.find(key_t{row_beg, row_num, col_beg, col_num});
        if (found == m_blocks.end()) {
            // mat_t(1, 1) would be a scalar: blocks are built at 2x2 or larger, then viewed
            const int R = std::max(row_num, 2), C = std::max(col_num, 2);
            mat_t<val_type> blk(R, C);
            for (int r = 0; r < R; ++r)
                for (int c = 0; c < C; ++c) blk(r, c) = entry(row_beg + r, col_beg + c);
            found = m_blocks.emplace(key_t{row_beg, row_num, col_beg, col_num}, std::move(blk)).first;
        }
        return found->second.view(0, 0, row_num, col_num);
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
