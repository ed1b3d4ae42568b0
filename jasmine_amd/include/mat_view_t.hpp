// mat_view_t: non-owning window / transposition of a mat_t (mat_view_t.hpp:7-135 of the
// reference).  Element (row, col) of the view is element
//   transposed ? (col + col_offset, row + row_offset) : (row + row_offset, col + col_offset)
// of the underlying matrix, which then applies its own modulo broadcast -- exactly the
// reference's mapping, including its swapped offsets under transposition.  On the device a
// view is a jas_leaf with those offsets, so views feed kernels without being copied.
#ifndef __MAT_VIEW_T_HPP__
#define __MAT_VIEW_T_HPP__
#include "mat_concepts.hpp"
#include "mat_t.hpp"
#include "mat_utility.hpp"

namespace jas {
// defined in mat_express_t.hpp: materialise any expression / view into a row-major mat_t
template <typename E>
auto materialize(const E &e);
} // namespace jas

template <typename agent_type>
class mat_view_t
{
public:
    using val_type = typename agent_type::ele_type;
    using ele_type = val_type;

private:
    agent_type &m_mat;
    int m_row_offset;
    int m_col_offset;
    int m_row_size;
    int m_col_size;
    bool m_transposed;

public:
    mat_view_t(agent_type &m, int row_offset = 0, int col_offset = 0, int row_size = -1, int col_size = -1) noexcept
        : m_mat(m), m_row_offset(row_offset), m_col_offset(col_offset), m_row_size(row_size), m_col_size(col_size),
          m_transposed(false)
    {
        m_row_size = (row_size == -1) ? m_mat.row_num() - row_offset : row_size;
        m_col_size = (col_size == -1) ? m_mat.col_num() - col_offset : col_size;
    }

    inline val_type operator()(int row, int col) const noexcept
    {
        const agent_type &m = m_mat;
        return m_transposed ? m(col + m_col_offset, row + m_row_offset) : m(row + m_row_offset, col + m_col_offset);
    }

    inline val_type &operator()(int row, int col) noexcept
    {
        return m_transposed ? m_mat(col + m_col_offset, row + m_row_offset)
                            : m_mat(row + m_row_offset, col + m_col_offset);
    }

    // write `other` through the view (mat_view_t.hpp:53-63), on the device
    template <typename other_type>
    void assign(const other_type &other)
    {
        auto src = jas::materialize(other);
        using S = typename decltype(src)::ele_type;
        if (src.is_scalar()) {  // broadcast a scalar by materialising it to the view's shape
            mat_t<S> full(row_num(), col_num());
            full = src(0, 0);
            src = std::move(full);
        }
        jas_leaf dst = leaf_mut();
        jas::check(jas_leaf_assign(src.device_data(), jas::dtype_of<S>(), row_num(), col_num(), &dst, nullptr));
    }

    inline int row_num() const noexcept { return m_transposed ? m_col_size : m_row_size; }
    inline int col_num() const noexcept { return m_transposed ? m_row_size : m_col_size; }

    std::string to_string() const
    {
        std::stringstream ss;
        ss << "matrix_view(" << row_num() << ", " << col_num() << ")";
        for (int i = 0; i < row_num(); ++i) {
            ss << "\n[ ";
            for (int j = 0; j < col_num(); ++j) ss << (*this)(i, j) << " ";
            ss << "]";
        }
        return ss.str();
    }

    inline mat_view_t<agent_type> t() const noexcept
    {
        mat_view_t<agent_type> mv(*this);
        mv.m_transposed = !m_transposed;
        return mv;
    }

    template <typename other_type>
    requires is_matrix<other_type>
    auto dot(const other_type &m) const;

    operator std::remove_const_t<agent_type>() const { return clone(); }

    mat_t<val_type> clone() const { return jas::materialize(*this); }

    // ---- device description ----
    agent_type &base() const noexcept { return m_mat; }
    int row_offset() const noexcept { return m_row_offset; }
    int col_offset() const noexcept { return m_col_offset; }
    bool transposed() const noexcept { return m_transposed; }
    jas_leaf leaf() const
    {
        jas_leaf l = m_mat.leaf();
        l.roff = m_row_offset;
        l.coff = m_col_offset;
        l.transposed = m_transposed ? 1 : 0;
        l.vrows = row_num();
        l.vcols = col_num();
        return l;
    }
    jas_leaf leaf_mut()
    {
        static_assert(!std::is_const_v<agent_type>, "cannot assign through a view of a const matrix");
        jas_leaf l = leaf();
        l.d_data = m_mat.device_data_mut();
        return l;
    }
};

// ---- mat_t's view factories (mat_view_t.hpp:137-243) ----
template <typename val_type>
requires jas::element_v<val_type>
mat_view_t<mat_t<val_type>> mat_t<val_type>::t() noexcept
{
    return mat_view_t<mat_t<val_type>>(*this).t();
}

template <typename val_type>
requires jas::element_v<val_type>
mat_view_t<mat_t<val_type>> mat_t<val_type>::view(int const &ro, int const &co, int const &rs, int const &cs) noexcept
{
    return mat_view_t<mat_t<val_type>>(*this, ro, co, rs, cs);
}

template <typename val_type>
requires jas::element_v<val_type>
mat_view_t<const mat_t<val_type>> mat_t<val_type>::view(int const &ro, int const &co, int const &rs,
                                                        int const &cs) const noexcept
{
    return mat_view_t<const mat_t<val_type>>(*this, ro, co, rs, cs);
}

#define JAS_VIEW_FACTORY(NAME, RO, CO, RS, CS)                                                                       \
    template <typename val_type>                                                                                     \
    requires jas::element_v<val_type>                                                                          \
    mat_view_t<mat_t<val_type>> mat_t<val_type>::NAME() noexcept                                                     \
    {                                                                                                                \
        return mat_view_t<mat_t<val_type>>(*this, RO, CO, RS, CS);                                                   \
    }                                                                                                                \
    template <typename val_type>                                                                                     \
    requires jas::element_v<val_type>                                                                          \
    mat_view_t<const mat_t<val_type>> mat_t<val_type>::NAME() const noexcept                                         \
    {                                                                                                                \
        return mat_view_t<const mat_t<val_type>>(*this, RO, CO, RS, CS);                                             \
    }
JAS_VIEW_FACTORY(back_col, 0, col_num() - 1, row_num(), 1)
JAS_VIEW_FACTORY(back_row, row_num() - 1, 0, 1, col_num())
JAS_VIEW_FACTORY(front_col, 0, 0, row_num(), 1)
JAS_VIEW_FACTORY(front_row, 0, 0, 1, col_num())
#undef JAS_VIEW_FACTORY

template <typename val_type>
requires jas::element_v<val_type>
mat_view_t<mat_t<val_type>> mat_t<val_type>::col(int const &idx) noexcept
{
    return mat_view_t<mat_t<val_type>>(*this, 0, idx, row_num(), 1);
}

template <typename val_type>
requires jas::element_v<val_type>
mat_view_t<const mat_t<val_type>> mat_t<val_type>::col(int const &idx) const noexcept
{
    return mat_view_t<const mat_t<val_type>>(*this, 0, idx, row_num(), 1);
}

template <typename val_type>
requires jas::element_v<val_type>
mat_view_t<mat_t<val_type>> mat_t<val_type>::row(int const &idx) noexcept
{
    return mat_view_t<mat_t<val_type>>(*this, idx, 0, 1, col_num());
}

template <typename val_type>
requires jas::element_v<val_type>
mat_view_t<const mat_t<val_type>> mat_t<val_type>::row(int const &idx) const noexcept
{
    return mat_view_t<const mat_t<val_type>>(*this, idx, 0, 1, col_num());
}

#include "mat_express_t.hpp"

#endif
