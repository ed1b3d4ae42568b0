// mat_t<T>: jasmine's owning dense 2-D matrix (mat_t.hpp:15-381 of the reference) with its
// storage in MI355X HBM.
//
// Same contract as the reference: value semantics (deep copy, pointer-stealing move),
// a 1x1 matrix is a scalar, construction zero-fills, element access broadcasts by modulo
// (operator()(r, c) reads element (r % rows, c % cols)), row- or column-major storage.
// The data lives in a device buffer; a host mirror is synchronised lazily, only when code
// touches elements through operator() or prints.  Device kernels (expression evaluation,
// GEMM, norms, attention) read and write the device copy directly.
#ifndef _MAT_T_HPP_
#define _MAT_T_HPP_
#include <algorithm>
#include <initializer_list>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "jasmine_hip.hpp"
#include "mat_utility.hpp"

template <typename val_type>
class mat_view_t;

template <typename val_type>
requires jas::element_v<val_type>
class mat_t
{
    template <typename U>
    requires jas::element_v<U>
    friend class mat_t;

public:
    using ele_type = val_type;
    struct device_uninit_tag {};

private:
    int m_rows = 0, m_cols = 0;
    bool m_row_first = true;
    bool m_scalar = false;
    bool m_alloc = false;  // jasmine's m_data != nullptr
    val_type m_scalar_val{};
    mutable std::vector<val_type> m_host;
    mutable jas::device_buffer m_dev;
    mutable bool m_host_ok = true, m_dev_ok = false;
    uint64_t m_stamp = jas::next_stamp();  // renewed on every change of the contents

    void touch() noexcept { m_stamp = jas::next_stamp(); }

    size_t count() const { return (size_t)m_rows * (size_t)m_cols; }

    void init_scalar(val_type v)
    {
        touch();
        m_scalar = true;
        m_alloc = true;
        m_scalar_val = v;
        m_rows = m_cols = 1;
        m_host.clear();
        m_dev.release();
        m_host_ok = true;
        m_dev_ok = false;
    }

    // zero-filled rows x cols (mat_t.hpp:53-69): zeros on the host, device copy on demand
    void init_matrix(int rows, int cols, bool row_first)
    {
        touch();
        m_scalar = false;
        m_alloc = true;
        m_rows = rows;
        m_cols = cols;
        m_row_first = row_first;
        m_host.assign(count(), val_type{});
        m_dev.release();
        m_host_ok = true;
        m_dev_ok = false;
    }

    void copy_from(const mat_t &m)
    {
        touch();
        m_row_first = m.m_row_first;
        if (m.m_scalar) {
            init_scalar(m.m_scalar_val);
            return;
        }
        m_scalar = false;
        m_alloc = m.m_alloc;
        m_rows = m.m_rows;
        m_cols = m.m_cols;
        if (m.m_dev_ok && jas::device_type<val_type>) {  // device-resident: copy on the device
            m_dev.allocate(count() * sizeof(val_type));
            jas::check(jas_memcpy_d2d(m_dev.get(), m.m_dev.get(), count() * sizeof(val_type), nullptr));
            m_dev_ok = true;
            m_host_ok = false;
            m_host.clear();
        } else {
            m.host_sync();
            m_host = m.m_host;
            m_host_ok = true;
            m_dev_ok = false;
            m_dev.release();
        }
    }

    void move_from(mat_t &m) noexcept
    {
        touch();
        m.touch();
        m_rows = m.m_rows, m_cols = m.m_cols, m_row_first = m.m_row_first;
        m_scalar = m.m_scalar, m_alloc = m.m_alloc, m_scalar_val = m.m_scalar_val;
        m_host = std::move(m.m_host);
        m_dev = std::move(m.m_dev);
        m_host_ok = m.m_host_ok, m_dev_ok = m.m_dev_ok;
        m.m_rows = m.m_cols = 0;
        m.m_alloc = false;
        m.m_scalar = false;
        m.m_host.clear();
        m.m_host_ok = true;
        m.m_dev_ok = false;
    }

public:
    mat_t() noexcept = default;

    mat_t(const ele_type &val) noexcept { init_scalar(val); }

    mat_t(int rows, int cols, bool row_first = true)
    {
        m_row_first = row_first;
        if (rows != 1 || cols != 1) init_matrix(rows, cols, row_first);
        else init_scalar(val_type{});
    }

    mat_t(const int &rows, const int &cols, std::initializer_list<val_type> l)
    {
        if (rows != 1 || cols != 1) {
            init_matrix(rows, cols, true);
            std::copy(l.begin(), l.begin() + std::min(l.size(), count()), m_host.begin());
        } else {
            init_scalar(*l.begin());
        }
    }

    // a row-major matrix whose device buffer a kernel is about to write (no host zero-fill)
    mat_t(int rows, int cols, device_uninit_tag)
    {
        m_rows = rows, m_cols = cols, m_row_first = true, m_alloc = true;
        if (rows == 1 && cols == 1) {
            init_scalar(val_type{});
            return;
        }
        m_dev.allocate(count() * sizeof(val_type));
        m_host_ok = false;
        m_dev_ok = true;
    }

    mat_t(mat_t &&m) noexcept { move_from(m); }
    mat_t &operator=(mat_t &&m) noexcept
    {
        if (this != &m) move_from(m);
        return *this;
    }
    mat_t(const mat_t &m) { copy_from(m); }
    mat_t &operator=(const mat_t &m)
    {
        if (this != &m) copy_from(m);
        return *this;
    }

    // fill every element (mat_t.hpp:162-174)
    template <typename scalar_type>
    requires std::is_arithmetic_v<scalar_type>
    mat_t &operator=(scalar_type s);

    // element-type conversion (mat_t.hpp:196-247): converted on the device when both types
    // are device types, element by element on the host otherwise
    template <typename other_val_type>
    requires std::is_convertible_v<other_val_type, val_type>
    mat_t(const mat_t<other_val_type> &m);

    template <typename other_val_type>
    requires std::is_convertible_v<other_val_type, val_type>
    mat_t &operator=(const mat_t<other_val_type> &m)
    {
        mat_t tmp(m);
        *this = std::move(tmp);
        return *this;
    }

    ~mat_t() = default;

    bool is_scalar() const noexcept { return m_scalar; }
    int row_num() const noexcept { return m_rows; }
    int col_num() const noexcept { return m_cols; }
    bool row_first() const noexcept { return m_row_first; }
    std::tuple<int, int> shape() const noexcept { return std::make_tuple(row_num(), col_num()); }
    bool valid() const noexcept { return m_alloc; }
    // identifies the current contents: changes whenever they may have changed (a write
    // through a reference kept from operator() after a later stamp() is not seen)
    uint64_t stamp() const noexcept { return m_stamp; }

    // mat_t.hpp:280-300: 1x1 becomes a scalar holding element (0,0); a different element
    // count re-allocates a zero row-major matrix; the same count keeps the matrix as is
    void reshape(int rows, int cols)
    {
        if (rows == 1 && cols == 1) {
            if (!m_scalar) {
                val_type v = count() ? (*this)(0, 0) : val_type{};
                init_scalar(v);
            }
        } else if ((long)rows * cols != (long)row_num() * col_num()) {
            init_matrix(rows, cols, true);
        }
    }

    // ---- storage access ----
    void host_sync() const
    {
        if (m_scalar || m_host_ok) return;
        m_host.resize(count());
        if (m_dev_ok && count())
            jas::check(jas_memcpy_d2h(m_host.data(), m_dev.get(), count() * sizeof(val_type), nullptr));
        m_host_ok = true;
    }
    // device pointer with current contents (uploads the host mirror if it is newer)
    const val_type *device_data() const
    {
        static_assert(jas::device_type<val_type>, "element type has no device representation (use float, double or int)");
        if (m_scalar) {  // scalars live on the host; materialise one element on demand
            m_dev.allocate(sizeof(val_type));
            jas::check(jas_memcpy_h2d(m_dev.get(), &m_scalar_val, sizeof(val_type), nullptr));
            return (const val_type *)m_dev.get();
        }
        if (!m_dev_ok) {
            m_dev.allocate(std::max<size_t>(count(), 1) * sizeof(val_type));
            if (count()) jas::check(jas_memcpy_h2d(m_dev.get(), m_host.data(), count() * sizeof(val_type), nullptr));
            m_dev_ok = true;
        }
        return (const val_type *)m_dev.get();
    }
    // device pointer for a kernel that overwrites the matrix (the host mirror goes stale)
    val_type *device_data_mut()
    {
        const val_type *p = device_data();
        if (!m_scalar) m_host_ok = false;
        touch();
        return const_cast<val_type *>(p);
    }
    // the jas_leaf describing this matrix as an expression operand
    jas_leaf leaf() const
    {
        jas_leaf l{};
        l.d_data = device_data();
        l.dtype = jas::dtype_of<val_type>();
        l.rows = m_rows;
        l.cols = m_cols;
        l.row_first = m_row_first ? 1 : 0;
        l.vrows = m_rows;
        l.vcols = m_cols;
        return l;
    }

    // ---- element access with jasmine's modulo broadcast (mat_t.hpp:302-320) ----
    val_type &operator()(int r, int c)
    {
        touch();
        if (m_scalar) return m_scalar_val;
        host_sync();
        m_dev_ok = false;  // the caller may write through the reference
        const int i = r % row_num(), j = c % col_num();
        return m_row_first ? m_host[(size_t)i * m_cols + j] : m_host[(size_t)j * m_rows + i];
    }
    const val_type &operator()(int r, int c) const
    {
        if (m_scalar) return m_scalar_val;
        host_sync();
        const int i = r % row_num(), j = c % col_num();
        return m_row_first ? m_host[(size_t)i * m_cols + j] : m_host[(size_t)j * m_rows + i];
    }

    std::string to_string() const
    {
        std::stringstream ss;
        ss << "matrix(" << row_num() << ", " << col_num() << ")";
        for (int i = 0; i < row_num(); ++i) {
            ss << "\n[ ";
            for (int j = 0; j < col_num(); ++j) ss << (*this)(i, j) << " ";
            ss << "]";
        }
        return ss.str();
    }

    mat_view_t<mat_t<val_type>> t() noexcept;
    mat_view_t<mat_t<val_type>> view(int const &row_offset = 0, int const &col_offset = 0, int const &row_size = -1,
                                     int const &col_size = -1) noexcept;
    mat_view_t<const mat_t<val_type>> view(int const &row_offset = 0, int const &col_offset = 0,
                                           int const &row_size = -1, int const &col_size = -1) const noexcept;
    mat_view_t<mat_t<val_type>> col(int const &col_num) noexcept;
    mat_view_t<const mat_t<val_type>> col(int const &col_num) const noexcept;
    mat_view_t<mat_t<val_type>> row(int const &row_num) noexcept;
    mat_view_t<const mat_t<val_type>> row(int const &row_num) const noexcept;
    mat_view_t<mat_t<val_type>> back_col() noexcept;
    mat_view_t<const mat_t<val_type>> back_col() const noexcept;
    mat_view_t<mat_t<val_type>> back_row() noexcept;
    mat_view_t<const mat_t<val_type>> back_row() const noexcept;
    mat_view_t<mat_t<val_type>> front_col() noexcept;
    mat_view_t<const mat_t<val_type>> front_col() const noexcept;
    mat_view_t<mat_t<val_type>> front_row() noexcept;
    mat_view_t<const mat_t<val_type>> front_row() const noexcept;

    // in-place transpose (mat_t.hpp:359-371)
    mat_t<val_type> &t_();

    mat_t<val_type> clone() const { return mat_t<val_type>(*this); }

    template <typename other_type>
    requires is_matrix<other_type>
    auto dot(const other_type &m) const;
};

// views and the expression engine complete mat_t's interface (t(), view(), dot(), ...)
#include "mat_view_t.hpp"

#endif
