// Expression templates of jasmine's API (mat_express_t.hpp:35-813 of the reference), lowered
// to the MI355X kernels.
//
// Operators (+ - * / > <), exp, sigmoid (and tanh, gelu, silu, which jasmine lacks) build a
// lazy tree exactly as in the reference: node ele_type is the std::common_type of the
// operands' types, a scalar operand keeps its own type, shapes broadcast by jasmine's
// modulo rule.  Evaluation happens at clone() / conversion to mat_t: the tree is serialised
// into one postfix program (Sethi-Ullman order) and evaluated by ONE fused kernel
// (jas_ew_eval).  mat_dot_t runs on the fp32 / fp64 MFMA GEMMs.  Reductions, softmax and
// hsoftmax run on the reduction kernels.
//
// Unlike the reference, expression nodes hold sub-expressions by value (matrices by
// reference), so `auto e = A * B + A;` stays valid after the full-expression.
#ifndef __MAT_EXPRESS_T_HPP__
#define __MAT_EXPRESS_T_HPP__
#include <cmath>
#include <limits>
#include <memory>
#include <numeric>
#include <sstream>
#include <string>
#include <tuple>
#include <vector>

#include "mat_concepts.hpp"
#include "mat_view_t.hpp"

template <typename lval_type, typename rval_type>
requires is_matrix<lval_type> && is_matrix<rval_type>
auto dot(lval_type const &lval, rval_type const &rval);

namespace jas {
namespace detail {

struct expr_tag {};

template <typename T>
struct is_mat : std::false_type {};
template <typename T>
struct is_mat<mat_t<T>> : std::true_type {};
template <typename T>
struct is_view : std::false_type {};
template <typename A>
struct is_view<mat_view_t<A>> : std::true_type {};

template <typename T>
constexpr bool is_mat_v = is_mat<std::remove_cv_t<T>>::value;
template <typename T>
constexpr bool is_view_v = is_view<std::remove_cv_t<T>>::value;
template <typename T>
constexpr bool is_node_v = std::is_base_of_v<expr_tag, T>;

template <typename T, bool = std::is_arithmetic_v<T>>
struct ele_of_impl {
    using type = T;
};
template <typename T>
struct ele_of_impl<T, false> {
    using type = typename T::ele_type;
};
template <typename T>
using ele_of = typename ele_of_impl<T>::type;

// operands: scalars by value, matrices by reference, views and nodes by value
template <typename T>
using store_t = std::conditional_t<is_mat_v<T>, const T &, T>;

// node arithmetic type code of a C++ element type
template <typename T>
constexpr int code_of()
{
    if constexpr (std::is_same_v<T, jas::bf16>) return JAS_BF16;
    else if constexpr (std::is_same_v<T, float>) return JAS_F32;
    else if constexpr (std::is_floating_point_v<T>) return JAS_F64;
    else return JAS_I32;
}

struct program {
    std::vector<jas_ew_ins> ins;
    std::vector<jas_leaf> leaves;
    std::vector<std::shared_ptr<void>> keep;  // temporaries that back leaves
};

template <typename T>
int rows_of(const T &x)
{
    if constexpr (std::is_arithmetic_v<T>) return 1;
    else return x.row_num();
}
template <typename T>
int cols_of(const T &x)
{
    if constexpr (std::is_arithmetic_v<T>) return 1;
    else return x.col_num();
}

// register need / leaf count / instruction count of an operand
template <typename T>
int need_of(const T &x)
{
    if constexpr (is_node_v<T>) return x.jas_need();
    else return 1;
}
template <typename T>
int leaves_of(const T &x)
{
    if constexpr (is_node_v<T>) return x.jas_leaves();
    else if constexpr (std::is_arithmetic_v<T>) return 0;
    else if constexpr (is_mat_v<T>) return x.is_scalar() ? 0 : 1;
    else return 1;
}
template <typename T>
int ins_of(const T &x)
{
    if constexpr (is_node_v<T>) return x.jas_ins();
    else return 1;
}

inline void push(program &p, int op, int dtype, int arg, double imm)
{
    jas_ew_ins i{};
    i.op = op;
    i.dtype = dtype;
    i.arg = arg;
    i.imm = imm;
    p.ins.push_back(i);
}

template <typename T>
void emit(const T &x, program &p, int budget);

} // namespace detail

template <typename E>
mat_t<detail::ele_of<E>> materialize_as(const E &e, int rows, int cols);

template <typename E>
auto materialize(const E &e)
{
    using T = detail::ele_of<E>;
    if constexpr (detail::is_mat_v<E>) {
        return mat_t<T>(e);
    } else if constexpr (requires { e.evaluate(); }) {  // mat_dot_t: the GEMM result
        return mat_t<T>(e.evaluate());
    } else if constexpr (detail::is_node_v<E> || detail::is_view_v<E>) {
        return materialize_as(e, e.row_num(), e.col_num());
    } else {  // a foreign is_matrix type: read it element by element through its operator()
        mat_t<T> m(e.row_num(), e.col_num());
        for (int i = 0; i < e.row_num(); ++i)
            for (int j = 0; j < e.col_num(); ++j) m(i, j) = e(i, j);
        return m;
    }
}

namespace detail {

// push operand x onto the program within `budget` stack slots; subtrees that would not fit
// (stack, leaves or instructions) are materialised first and enter as a leaf
template <typename T>
void emit(const T &x, program &p, int budget)
{
    if constexpr (std::is_arithmetic_v<T>) {
        push(p, JAS_OP_CONST, code_of<T>(), 0, (double)x);
    } else if constexpr (is_mat_v<T>) {
        using E = typename T::ele_type;
        if (x.is_scalar()) {
            push(p, JAS_OP_CONST, code_of<E>(), 0, (double)x(0, 0));
        } else {
            p.leaves.push_back(x.leaf());
            push(p, JAS_OP_LEAF, code_of<E>(), (int)p.leaves.size() - 1, 0.0);
        }
    } else if constexpr (is_view_v<T>) {
        p.leaves.push_back(x.leaf());
        push(p, JAS_OP_LEAF, code_of<typename T::ele_type>(), (int)p.leaves.size() - 1, 0.0);
    } else {
        const bool fits = !is_node_v<T> ? false
                                        : (need_of(x) <= budget &&
                                           (int)p.leaves.size() + leaves_of(x) <= JAS_EW_MAX_LEAVES &&
                                           (int)p.ins.size() + ins_of(x) <= JAS_EW_MAX_INS - 2);
        if constexpr (is_node_v<T>) {
            if (fits && !x.jas_opaque()) {
                x.jas_emit(p, budget);
                return;
            }
        }
        auto m = std::make_shared<mat_t<ele_of<T>>>(materialize(x));
        p.keep.push_back(m);
        emit(*m, p, budget);
    }
}

// binary / unary expression nodes
template <typename Derived, typename L, typename R, int OP>
class binary_node : public expr_tag
{
public:
    using lval_base_type = ele_of<L>;
    using rval_base_type = ele_of<R>;
    using ele_type = std::common_type_t<lval_base_type, rval_base_type>;

    binary_node(L const &l, R const &r) : m_left(l), m_right(r) {}

    int row_num() const { return std::max(rows_of<L>(m_left), rows_of<R>(m_right)); }
    int col_num() const { return std::max(cols_of<L>(m_left), cols_of<R>(m_right)); }
    std::tuple<int, int> shape() const { return std::make_tuple(row_num(), col_num()); }

    // element access materialises the tree once (value semantics, cached)
    ele_type operator()(int i, int j) const { return cached()(i, j); }

    std::string to_string() const
    {
        std::stringstream ss;
        const auto &m = cached();
        ss << Derived::type_name() << "(" << row_num() << ", " << col_num() << ")";
        for (int i = 0; i < row_num(); ++i) {
            ss << "\n[ ";
            for (int j = 0; j < col_num(); ++j) ss << m(i, j) << " ";
            ss << " ]";
        }
        return ss.str();
    }

    mat_t<ele_type> clone() const { return jas::materialize(static_cast<const Derived &>(*this)); }
    operator mat_t<ele_type>() const { return clone(); }

    template <typename other_type>
    auto dot(const other_type &m) const;

    int jas_need() const
    {
        int l = need_of(m_left), r = need_of(m_right);
        return l == r ? l + 1 : std::max(l, r);
    }
    int jas_leaves() const { return leaves_of(m_left) + leaves_of(m_right); }
    int jas_ins() const { return ins_of(m_left) + ins_of(m_right) + 1; }
    bool jas_opaque() const { return false; }
    void jas_emit(program &p, int budget) const
    {
        const bool swap = need_of(m_right) > need_of(m_left);
        if (swap) {
            emit(m_right, p, budget);
            emit(m_left, p, budget - 1);
        } else {
            emit(m_left, p, budget);
            emit(m_right, p, budget - 1);
        }
        push(p, OP, code_of<ele_type>(), swap ? 1 : 0, 0.0);
    }

protected:
    store_t<L> m_left;
    store_t<R> m_right;
    mutable std::shared_ptr<mat_t<ele_type>> m_cache;
    const mat_t<ele_type> &cached() const
    {
        if (!m_cache) m_cache = std::make_shared<mat_t<ele_type>>(clone());
        return *m_cache;
    }
};

template <typename Derived, typename V, int OP, typename OutT = ele_of<V>>
class unary_node : public expr_tag
{
public:
    using val_base_type = ele_of<V>;
    using ele_type = OutT;

    explicit unary_node(V const &v, double imm = 0.0) : m_val(v), m_imm(imm) {}

    int row_num() const { return rows_of<V>(m_val); }
    int col_num() const { return cols_of<V>(m_val); }
    std::tuple<int, int> shape() const { return std::make_tuple(row_num(), col_num()); }
    ele_type operator()(int i, int j) const { return cached()(i, j); }

    std::string to_string() const
    {
        std::stringstream ss;
        const auto &m = cached();
        ss << Derived::type_name() << "(" << row_num() << ", " << col_num() << ")";
        for (int i = 0; i < row_num(); ++i) {
            ss << "\n[ ";
            for (int j = 0; j < col_num(); ++j) ss << m(i, j) << " ";
            ss << " ]";
        }
        return ss.str();
    }

    mat_t<ele_type> clone() const { return jas::materialize(static_cast<const Derived &>(*this)); }
    operator mat_t<ele_type>() const { return clone(); }

    template <typename other_type>
    auto dot(const other_type &m) const;

    int jas_need() const { return need_of(m_val); }
    int jas_leaves() const { return leaves_of(m_val); }
    int jas_ins() const { return ins_of(m_val) + 1; }
    bool jas_opaque() const { return false; }
    void jas_emit(program &p, int budget) const
    {
        emit(m_val, p, budget);
        push(p, OP, code_of<ele_type>(), 0, m_imm);
    }

protected:
    store_t<V> m_val;
    double m_imm;
    mutable std::shared_ptr<mat_t<ele_type>> m_cache;
    const mat_t<ele_type> &cached() const
    {
        if (!m_cache) m_cache = std::make_shared<mat_t<ele_type>>(clone());
        return *m_cache;
    }
};

} // namespace detail

// materialise an expression over an explicit output shape (the += loops use the left
// operand's shape), evaluated by one jas_ew_eval launch
template <typename E>
mat_t<detail::ele_of<E>> materialize_as(const E &e, int rows, int cols)
{
    using T = detail::ele_of<E>;
    static_assert(jas::device_type<T>, "expression element type has no device representation");
    detail::program p;
    detail::emit(e, p, JAS_EW_MAX_STACK);
    if (rows == 1 && cols == 1) {  // a 1x1 result is a scalar mat_t (mat_t.hpp:83-94)
        device_buffer tmp(sizeof(T));
        check(jas_ew_eval(p.ins.data(), (int)p.ins.size(), p.leaves.data(), (int)p.leaves.size(), tmp.get(),
                          dtype_of<T>(), 1, 1, nullptr));
        T v{};
        check(jas_memcpy_d2h(&v, tmp.get(), sizeof(T), nullptr));
        return mat_t<T>(v);
    }
    mat_t<T> out(rows, cols, typename mat_t<T>::device_uninit_tag{});
    check(jas_ew_eval(p.ins.data(), (int)p.ins.size(), p.leaves.data(), (int)p.leaves.size(), out.device_data_mut(),
                      dtype_of<T>(), rows, cols, nullptr));
    return out;
}

// a row-major dense mat_t<T> with the contents of x (no copy when x already is one)
template <typename T, typename E>
std::shared_ptr<const mat_t<T>> as_dense(const E &x)
{
    if constexpr (detail::is_mat_v<E> && std::is_same_v<detail::ele_of<E>, T>) {
        if (x.row_first() || x.row_num() == 1 || x.col_num() == 1)  // vectors are layout-free
            return std::shared_ptr<const mat_t<T>>(&x, [](const mat_t<T> *) {});
    }
    if constexpr (std::is_same_v<detail::ele_of<E>, T>) return std::make_shared<const mat_t<T>>(materialize(x));
    else return std::make_shared<const mat_t<T>>(mat_t<T>(materialize(x)));
}

// a GEMM operand: device pointer plus (row, col) element strides; mat_t and affine views
// are used in place, anything else is materialised row-major first
template <typename T>
struct gemm_operand_t {
    const T *p;
    long s0, s1;
    std::shared_ptr<const void> hold;
};

template <typename T, typename X>
gemm_operand_t<T> gemm_operand(const X &x)
{
    using XT = typename X::ele_type;
    if constexpr (std::is_same_v<XT, T> && detail::is_mat_v<X>) {
        if (!x.is_scalar()) {
            if (x.row_first()) return {x.device_data(), (long)x.col_num(), 1, nullptr};
            return {x.device_data(), 1, (long)x.row_num(), nullptr};
        }
    }
    if constexpr (std::is_same_v<XT, T> && detail::is_view_v<X>) {
        // jasmine's view mapping is affine unless the underlying modulo wraps
        const auto &m = x.base();
        const int R = m.row_num(), C = m.col_num();
        const long ra = m.row_first() ? C : 1, cb = m.row_first() ? 1 : R;  // strides of (a, b)
        const bool t = x.transposed();
        const long amax = t ? (long)x.col_num() - 1 + x.col_offset() : (long)x.row_num() - 1 + x.row_offset();
        const long bmax = t ? (long)x.row_num() - 1 + x.row_offset() : (long)x.col_num() - 1 + x.col_offset();
        if (!m.is_scalar() && amax < R && bmax < C) {
            const long a0 = t ? x.col_offset() : x.row_offset(), b0 = t ? x.row_offset() : x.col_offset();
            const T *base = m.device_data() + a0 * ra + b0 * cb;
            return t ? gemm_operand_t<T>{base, cb, ra, nullptr} : gemm_operand_t<T>{base, ra, cb, nullptr};
        }
    }
    auto d = as_dense<T>(x);
    if (d->is_scalar()) {  // a 1x1 operand: keep a one-element device copy alive
        auto h = std::make_shared<device_buffer>(sizeof(T));
        const T v = (*d)(0, 0);
        check(jas_memcpy_h2d(h->get(), &v, sizeof(T), nullptr));
        return {(const T *)h->get(), 1, 1, h};
    }
    return {d->device_data(), (long)d->col_num(), 1, d};
}

} // namespace jas

// ---------------------------------------------------------------- binary nodes
#define JAS_BINARY_NODE(NAME, OP, SYM)                                                                             \
    template <typename lval_type, typename rval_type>                                                              \
    class NAME : public jas::detail::binary_node<NAME<lval_type, rval_type>, lval_type, rval_type, OP>             \
    {                                                                                                              \
    public:                                                                                                        \
        using base_type = jas::detail::binary_node<NAME<lval_type, rval_type>, lval_type, rval_type, OP>;          \
        using base_type::base_type;                                                                                \
        static std::string type_name() { return #NAME; }                                                           \
    };                                                                                                             \
    template <typename lval_type, typename rval_type>                                                              \
    requires is_caculable<lval_type, rval_type> &&                                                                 \
             (is_matrix<lval_type> || is_matrix<rval_type>)                                                        \
    auto operator SYM(lval_type const &left, rval_type const &right)                                               \
    {                                                                                                              \
        return NAME<lval_type, rval_type>(left, right);                                                            \
    }

JAS_BINARY_NODE(mat_greater_t, JAS_OP_GT, >)   // mat_express_t.hpp:119-151
JAS_BINARY_NODE(mat_less_t, JAS_OP_LT, <)      // :153-186
JAS_BINARY_NODE(mat_add_t, JAS_OP_ADD, +)      // :188-223
JAS_BINARY_NODE(mat_sub_t, JAS_OP_SUB, -)      // :253-286
JAS_BINARY_NODE(mat_mul_t, JAS_OP_MUL, *)      // :288-321
JAS_BINARY_NODE(mat_div_t, JAS_OP_DIV, /)      // :323-358
#undef JAS_BINARY_NODE

// left(i, j) += right(i, j) over left's shape (mat_express_t.hpp:225-251)
template <typename lval_type, typename rval_type>
requires is_matrix<lval_type> && (is_matrix<rval_type> || std::is_arithmetic_v<rval_type>)
decltype(auto) operator+=(lval_type &left, rval_type const &right)
{
    using LT = typename lval_type::ele_type;
    auto sum = jas::materialize_as(left + right, left.row_num(), left.col_num());
    if constexpr (jas::detail::is_mat_v<lval_type>) left = mat_t<LT>(sum);
    else left.assign(sum);
    return left;
}

// ---------------------------------------------------------------- unary nodes
#define JAS_UNARY_NODE(NAME, OP, FN, DOC)                                                                          \
    template <typename val_type>                                                                                   \
    class NAME : public jas::detail::unary_node<NAME<val_type>, val_type, OP>                                      \
    {                                                                                                              \
    public:                                                                                                        \
        using base_type = jas::detail::unary_node<NAME<val_type>, val_type, OP>;                                   \
        explicit NAME(val_type const &v) : base_type(v) {}                                                         \
        static std::string type_name() { return #NAME; }                                                           \
    };                                                                                                             \
    template <typename val_type>                                                                                   \
    requires is_matrix<val_type>                                                                                   \
    auto FN(val_type const &val)                                                                                   \
    {                                                                                                              \
        return NAME<val_type>(val);                                                                                \
    }

JAS_UNARY_NODE(mat_exp_t, JAS_OP_EXP, exp, "mat_express_t.hpp:439-469")
JAS_UNARY_NODE(mat_sigmoid_t, JAS_OP_SIGMOID, sigmoid, "mat_express_t.hpp:479-509")
JAS_UNARY_NODE(mat_tanh_t, JAS_OP_TANH, tanh, "new: tanh in the operand type")
JAS_UNARY_NODE(mat_gelu_t, JAS_OP_GELU, gelu, "new: GPT-2 tanh GELU")
JAS_UNARY_NODE(mat_silu_t, JAS_OP_SILU, silu, "new: x * sigmoid(x)")
#undef JAS_UNARY_NODE

// scalar sigmoid (mat_express_t.hpp:471-476)
template <typename val_type>
requires std::is_arithmetic_v<val_type>
val_type sigmoid(val_type const &val)
{
    return 1.0 / (1.0 + std::exp(-val));
}

// ---------------------------------------------------------------- matrix product
template <typename lval_type, typename rval_type>
requires is_matrix<lval_type> && is_matrix<rval_type>
class mat_dot_t : public jas::detail::expr_tag
{
public:
    using ele_type = std::common_type_t<typename lval_type::ele_type, typename rval_type::ele_type>;

private:
    jas::detail::store_t<lval_type> m_lval;
    jas::detail::store_t<rval_type> m_rval;
    mutable std::shared_ptr<mat_t<ele_type>> m_cache;

public:
    mat_dot_t(lval_type const &lval, rval_type const &rval) : m_lval(lval), m_rval(rval)
    {
        if (lval.col_num() != rval.row_num())
            throw std::invalid_argument("mat_dot_t: inner dimensions do not match for dot product");
    }

    int row_num() const { return m_lval.row_num(); }
    int col_num() const { return m_rval.col_num(); }
    std::tuple<int, int> shape() const { return std::make_tuple(row_num(), col_num()); }

    ele_type operator()(int i, int j) const { return evaluate()(i, j); }

    template <typename other_type>
    auto dot(const other_type &m) const
    {
        return ::dot(*this, m);
    }

    std::string to_string() const
    {
        std::stringstream ss;
        const auto &m = evaluate();
        ss << "mat_dot_t(" << row_num() << ", " << col_num() << ")";
        for (int i = 0; i < row_num(); ++i) {
            ss << "\n[ ";
            for (int j = 0; j < col_num(); ++j) ss << m(i, j) << " ";
            ss << " ]";
        }
        return ss.str();
    }

    // C = A . B on the MFMA GEMM (fp32 or fp64)
    const mat_t<ele_type> &evaluate() const
    {
        if (m_cache) return *m_cache;
        if constexpr (std::is_same_v<ele_type, jas::bf16>) {
            // bf16 products: both operands widened exactly to float, fp32 MFMA GEMM with fp32
            // accumulation, the result rounded to bf16
            mat_t<float> af(jas::materialize(m_lval)), bf(jas::materialize(m_rval));
            mat_t<float> cf = ::dot(af, bf).clone();
            m_cache = std::make_shared<mat_t<ele_type>>(mat_t<ele_type>(cf));
            return *m_cache;
        }
        static_assert(std::is_same_v<ele_type, float> || std::is_same_v<ele_type, double> ||
                          std::is_same_v<ele_type, jas::bf16>,
                      "mat_dot_t runs on the fp32 / fp64 GEMM only");
        const int M = row_num(), N = col_num(), K = m_lval.col_num();
        auto a = jas::gemm_operand<ele_type>(m_lval);
        auto b = jas::gemm_operand<ele_type>(m_rval);
        jas::device_buffer tmp;
        mat_t<ele_type> out;
        ele_type *c;
        if (M == 1 && N == 1) {
            tmp.allocate(sizeof(ele_type));
            c = (ele_type *)tmp.get();
        } else {
            out = mat_t<ele_type>(M, N, typename mat_t<ele_type>::device_uninit_tag{});
            c = out.device_data_mut();
        }
        if constexpr (std::is_same_v<ele_type, float>)
            jas::check(jas_gemm(M, N, K, a.p, a.s0, a.s1, b.p, b.s0, b.s1, c, N, 1, nullptr, 0, JAS_ACT_NONE, 0, 1,
                                0, 0, 0, 0, nullptr));
        else if constexpr (std::is_same_v<ele_type, double>)
            jas::check(jas_gemm_f64(M, N, K, a.p, a.s0, a.s1, b.p, b.s0, b.s1, c, N, 1, nullptr, 0, nullptr));
        if (M == 1 && N == 1) {
            ele_type v{};
            jas::check(jas_memcpy_d2h(&v, c, sizeof(ele_type), nullptr));
            out = mat_t<ele_type>(v);
        }
        m_cache = std::make_shared<mat_t<ele_type>>(std::move(out));
        return *m_cache;
    }

    operator mat_t<ele_type>() const { return clone(); }
    mat_t<ele_type> clone() const { return evaluate(); }

    // inside a larger expression the product enters as one materialised leaf
    int jas_need() const { return 1; }
    int jas_leaves() const { return 1; }
    int jas_ins() const { return 1; }
    bool jas_opaque() const { return true; }
    void jas_emit(jas::detail::program &, int) const {}
};

template <typename lval_type, typename rval_type>
requires is_matrix<lval_type> && is_matrix<rval_type>
auto dot(lval_type const &lval, rval_type const &rval)
{
    return mat_dot_t<lval_type, rval_type>(lval, rval);
}

template <typename Derived, typename L, typename R, int OP>
template <typename other_type>
auto jas::detail::binary_node<Derived, L, R, OP>::dot(const other_type &m) const
{
    return ::dot(static_cast<const Derived &>(*this), m);
}

template <typename Derived, typename V, int OP, typename OutT>
template <typename other_type>
auto jas::detail::unary_node<Derived, V, OP, OutT>::dot(const other_type &m) const
{
    return ::dot(static_cast<const Derived &>(*this), m);
}

template <typename val_type>
requires jas::element_v<val_type>
template <typename other_type>
requires is_matrix<other_type>
auto mat_t<val_type>::dot(const other_type &m) const
{
    return ::dot(*this, m);
}

template <typename agent_type>
template <typename other_type>
requires is_matrix<other_type>
auto mat_view_t<agent_type>::dot(const other_type &m) const
{
    return ::dot(*this, m);
}

// ---------------------------------------------------------------- mat_t members needing kernels
template <typename val_type>
requires jas::element_v<val_type>
template <typename scalar_type>
requires std::is_arithmetic_v<scalar_type>
mat_t<val_type> &mat_t<val_type>::operator=(scalar_type s)
{
    touch();
    if (m_scalar) {
        m_scalar_val = static_cast<val_type>(s);
        return *this;
    }
    if constexpr (jas::device_type<val_type>) {
        if (count()) {  // one-instruction program: CONST in the element type
            jas_ew_ins in{};
            in.op = JAS_OP_CONST;
            in.dtype = jas::detail::code_of<val_type>();
            in.imm = (double)static_cast<val_type>(s);
            if (!m_dev_ok) m_dev.allocate(count() * sizeof(val_type));
            m_dev_ok = true;
            m_host_ok = false;
            jas::check(jas_ew_eval(&in, 1, nullptr, 0, m_dev.get(), jas::dtype_of<val_type>(), 1, (int)count(), nullptr));
        }
    } else {
        host_sync();
        std::fill(m_host.begin(), m_host.end(), static_cast<val_type>(s));
    }
    return *this;
}

template <typename val_type>
requires jas::element_v<val_type>
template <typename other_val_type>
requires std::is_convertible_v<other_val_type, val_type>
mat_t<val_type>::mat_t(const mat_t<other_val_type> &m)
{
    m_row_first = m.m_row_first;
    if (m.is_scalar()) {
        init_scalar(static_cast<val_type>(m.m_scalar_val));
        return;
    }
    if constexpr (jas::device_type<val_type> && jas::device_type<other_val_type>) {
        m_rows = m.m_rows, m_cols = m.m_cols, m_alloc = m.m_alloc, m_scalar = false;
        if (count()) {  // LEAF in the source type, stored converted (static_cast semantics)
            jas_leaf lf = m.leaf();
            lf.rows = 1, lf.cols = (int)count(), lf.row_first = 1, lf.vrows = 1, lf.vcols = (int)count();
            jas_ew_ins in{};
            in.op = JAS_OP_LEAF;
            in.dtype = jas::detail::code_of<other_val_type>();
            m_dev.allocate(count() * sizeof(val_type));
            m_dev_ok = true;
            m_host_ok = false;
            jas::check(jas_ew_eval(&in, 1, &lf, 1, m_dev.get(), jas::dtype_of<val_type>(), 1, (int)count(), nullptr));
        }
    } else {
        init_matrix(m.row_num(), m.col_num(), m.m_row_first);
        for (int i = 0; i < row_num(); ++i)
            for (int j = 0; j < col_num(); ++j) (*this)(i, j) = static_cast<val_type>(m(i, j));
    }
}

template <typename val_type>
requires jas::element_v<val_type>
mat_t<val_type> &mat_t<val_type>::t_()
{
    if (m_scalar) return *this;
    mat_t<val_type> m = jas::materialize(this->t());
    *this = std::move(m);
    return *this;
}

// ---------------------------------------------------------------- reductions
namespace jas::detail {
template <typename T, typename E>
mat_t<T> reduce_as(const E &val, int op, int axis);

// jas_reduce over any matrix operand; returns a device matrix of shape (rows_out, cols_out)
template <typename E>
mat_t<ele_of<E>> reduce(const E &val, int op, int axis)
{
    using T = ele_of<E>;
    if constexpr (std::is_same_v<T, jas::bf16>) {
        // bf16 operands are read as such and summed in float; the result is rounded to bf16
        mat_t<float> r = reduce_as<float>(val, op, axis);
        return mat_t<jas::bf16>(r);
    } else {
        return reduce_as<T>(val, op, axis);
    }
}

template <typename T, typename E>
mat_t<T> reduce_as(const E &val, int op, int axis)
{
    static_assert(std::is_same_v<T, float> || std::is_same_v<T, double>, "reductions run in float or double");
    std::shared_ptr<const void> hold;
    jas_leaf lf;
    if constexpr (is_mat_v<E> || is_view_v<E>) {
        lf = val.leaf();
        if constexpr (is_mat_v<E>)
            if (val.is_scalar()) lf.rows = lf.cols = lf.vrows = lf.vcols = 1;
    } else {
        auto m = std::make_shared<mat_t<ele_of<E>>>(materialize(val));
        lf = m->leaf();
        hold = m;
    }
    const int R = val.row_num(), C = val.col_num();
    const int orow = axis == 0 ? R : 1, ocol = axis == 1 ? C : 1;
    if (orow == 1 && ocol == 1) {
        device_buffer tmp(sizeof(T));
        check(jas_reduce(&lf, op, axis, tmp.get(), dtype_of<T>(), nullptr));
        T v{};
        check(jas_memcpy_d2h(&v, tmp.get(), sizeof(T), nullptr));
        return mat_t<T>(v);
    }
    mat_t<T> out(orow, ocol, typename mat_t<T>::device_uninit_tag{});
    check(jas_reduce(&lf, op, axis, out.device_data_mut(), dtype_of<T>(), nullptr));
    return out;
}
} // namespace jas::detail

// mat_express_t.hpp:511-628
template <typename val_type>
requires std::is_arithmetic_v<val_type>
auto sum(val_type const &val)
{
    return val;
}
template <typename val_type>
requires is_matrix<val_type>
auto sum(val_type const &val)
{
    return jas::detail::reduce(val, 0, 2)(0, 0);
}
template <typename val_type>
requires is_matrix<val_type>
auto vsum(val_type const &val)
{
    return jas::detail::reduce(val, 0, 1);
}
template <typename val_type>
requires is_matrix<val_type>
auto hsum(val_type const &val)
{
    return jas::detail::reduce(val, 0, 0);
}
template <typename val_type>
requires is_matrix<val_type>
auto vmean(val_type const &val)
{
    return jas::detail::reduce(val, 2, 1);
}
template <typename val_type>
requires is_matrix<val_type>
auto hmean(val_type const &val)
{
    return jas::detail::reduce(val, 2, 0);
}
template <typename val_type>
requires is_matrix<val_type>
auto mean(val_type const &val)
{
    return jas::detail::reduce(val, 2, 2)(0, 0);
}
template <typename input_type>
requires is_matrix<input_type>
auto max(input_type const &val)
{
    return jas::detail::reduce(val, 1, 2)(0, 0);
}
template <typename input_type>
requires is_matrix<input_type>
auto hmax(input_type const &val)
{
    return jas::detail::reduce(val, 1, 0);
}

// pow(mat, p) materialises std::pow(x, p) in the element type (mat_express_t.hpp:587-596)
template <typename input_type>
requires is_matrix<input_type>
auto pow(input_type const &val, double const p = 2.)
{
    using T = typename std::decay_t<input_type>::ele_type;
    struct pow_node : jas::detail::unary_node<pow_node, input_type, JAS_OP_POW> {
        pow_node(input_type const &v, double e) : jas::detail::unary_node<pow_node, input_type, JAS_OP_POW>(v, e) {}
        static std::string type_name() { return "pow"; }
    };
    return mat_t<T>(jas::materialize(pow_node(val, p)));
}

// sqrt(mat) materialises std::sqrt elementwise (mat_express_t.hpp:804-813)
template <typename val_type>
requires is_matrix<val_type>
auto sqrt(val_type const &val)
{
    using T = typename val_type::ele_type;
    struct sqrt_node : jas::detail::unary_node<sqrt_node, val_type, JAS_OP_SQRT> {
        explicit sqrt_node(val_type const &v) : jas::detail::unary_node<sqrt_node, val_type, JAS_OP_SQRT>(v) {}
        static std::string type_name() { return "sqrt"; }
    };
    return mat_t<T>(jas::materialize(sqrt_node(val)));
}

// ---------------------------------------------------------------- softmax
// row softmax (mat_express_t.hpp:681-694): float on the fused one-pass kernel; other types
// as jasmine's four passes (hmax, exp(x - max), hsum, divide) on the generic kernels
template <typename input_type>
auto hsoftmax(const input_type &input)
{
    using val_type = typename std::decay_t<input_type>::ele_type;
    if constexpr (std::is_same_v<val_type, float>) {
        auto x = jas::as_dense<float>(input);
        const int R = x->row_num(), C = x->col_num();
        if (R == 1 && C == 1) return mat_t<float>(1.0f);
        mat_t<float> y(R, C, mat_t<float>::device_uninit_tag{});
        jas::check(jas_softmax(x->device_data(), y.device_data_mut(), R, C, C, C, 1, nullptr));
        return y;
    } else {
        mat_t<val_type> max_val = hmax(input);
        mat_t<val_type> exp_val = exp(input - max_val);
        mat_t<val_type> sum_exp = hsum(exp_val);
        mat_t<val_type> softmax_val = exp_val / sum_exp;
        return softmax_val;
    }
}

// whole-matrix softmax (mat_softmax_t, mat_express_t.hpp:630-679)
template <typename val_type>
requires std::is_arithmetic_v<val_type>
auto softmax(val_type const &)
{
    return static_cast<val_type>(1.);
}
template <typename val_type>
requires is_matrix<val_type>
auto softmax(val_type const &val)
{
    using T = typename val_type::ele_type;
    if constexpr (std::is_same_v<T, float>) {
        auto x = jas::as_dense<float>(val);
        if (x->is_scalar()) return mat_t<float>(1.0f);
        mat_t<float> y(x->row_num(), x->col_num(), mat_t<float>::device_uninit_tag{});
        jas::check(jas_softmax_global(x->device_data(), y.device_data_mut(), (long)x->row_num() * x->col_num(), nullptr));
        return y;
    } else {
        T m = max(val);
        T s = sum(exp(val - m));
        return mat_t<T>(exp(val - m) / s);
    }
}

#endif
