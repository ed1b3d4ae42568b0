// C++ side of the boundary: status codes -> the exception types jasmine throws, RAII device
// buffers, element-type -> jas_dtype mapping.  Included by every jasmine-API header.
#ifndef JASMINE_AMD_JASMINE_HIP_HPP
#define JASMINE_AMD_JASMINE_HIP_HPP

#include <atomic>
#include <cstdint>
#include <cstring>
#include <ostream>
#include <stdexcept>
#include <string>
#include <type_traits>
#include <utility>

#include "../../include/jasmine_hip.h"

namespace jas {

// JAS_ERR_INVALID -> std::invalid_argument (mat_express_t.hpp:711), JAS_ERR_RANGE ->
// std::out_of_range (mat_RoPE_t.hpp:57), anything else -> std::runtime_error (mat_mha_t.hpp:240)
inline void check(jas_status s)
{
    if (s == JAS_OK) return;
    std::string m = jas_last_error();
    if (s == JAS_ERR_INVALID) throw std::invalid_argument(m);
    if (s == JAS_ERR_RANGE) throw std::out_of_range(m);
    throw std::runtime_error(m);
}

// A process-wide counter: every mat_t takes a fresh value whenever its contents may change,
// so (stamp) identifies one state of one matrix (caches key derived data on it).
inline uint64_t next_stamp() noexcept
{
    static std::atomic<uint64_t> counter{0};
    return counter.fetch_add(1, std::memory_order_relaxed) + 1;
}

inline void ensure_init()
{
    static bool done = false;
    if (!done) {
        check(jas_init(-1));
        done = true;
    }
}

// bf16 element type of mat_t<jas::bf16> (the reference gates mat_t on std::is_arithmetic_v,
// mat_t.hpp:15-16, which no 16-bit float type passes).  Storage is the upper half of an
// IEEE float; values convert to float exactly and from float round to nearest even (NaN
// stays a quiet NaN).  Arithmetic on bf16 matrices is float arithmetic rounded to bf16 per
// node, on the host and in the kernels alike.
struct bf16 {
    uint16_t bits = 0;
    constexpr bf16() = default;
    bf16(float f) : bits(from_float(f)) {}
    template <typename T>
    requires(std::is_arithmetic_v<T> && !std::is_same_v<T, float>)
    bf16(T v) : bf16(static_cast<float>(v)) {}
    operator float() const
    {
        const uint32_t u = (uint32_t)bits << 16;
        float f;
        std::memcpy(&f, &u, 4);
        return f;
    }
    static uint16_t from_float(float f)
    {
        uint32_t u;
        std::memcpy(&u, &f, 4);
        if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)(((u >> 16) & 0x8000u) | 0x7fc0u);
        return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
};
static_assert(sizeof(bf16) == 2 && std::is_trivially_copyable_v<bf16>, "bf16 is a 2-byte value");
inline std::ostream &operator<<(std::ostream &o, bf16 v) { return o << static_cast<float>(v); }

// element types mat_t accepts: jasmine's arithmetic types plus bf16
template <typename T>
constexpr bool element_v = std::is_arithmetic_v<T> || std::is_same_v<T, bf16>;

template <typename T>
constexpr int dtype_of()
{
    if constexpr (std::is_same_v<T, bf16>) return JAS_BF16;
    else if constexpr (std::is_same_v<T, float>) return JAS_F32;
    else if constexpr (std::is_same_v<T, double>) return JAS_F64;
    else if constexpr (std::is_integral_v<T> && sizeof(T) == 4 && std::is_signed_v<T>) return JAS_I32;
    else return -1;
}

template <typename T>
constexpr bool device_type = dtype_of<T>() >= 0;

// owning device allocation (moves only)
class device_buffer
{
    void *m_p = nullptr;
    size_t m_bytes = 0;

public:
    device_buffer() = default;
    explicit device_buffer(size_t bytes) { allocate(bytes); }
    device_buffer(const device_buffer &) = delete;
    device_buffer &operator=(const device_buffer &) = delete;
    device_buffer(device_buffer &&o) noexcept : m_p(o.m_p), m_bytes(o.m_bytes) { o.m_p = nullptr, o.m_bytes = 0; }
    device_buffer &operator=(device_buffer &&o) noexcept
    {
        if (this != &o) {
            release();
            m_p = o.m_p, m_bytes = o.m_bytes;
            o.m_p = nullptr, o.m_bytes = 0;
        }
        return *this;
    }
    ~device_buffer() { release(); }
    void allocate(size_t bytes)
    {
        if (bytes <= m_bytes && m_p) return;
        release();
        ensure_init();
        check(jas_pool_alloc(&m_p, bytes ? bytes : 1));
        m_bytes = bytes;
    }
    void release() noexcept
    {
        if (m_p) jas_pool_free(m_p);
        m_p = nullptr;
        m_bytes = 0;
    }
    void *get() const { return m_p; }
    size_t bytes() const { return m_bytes; }
};

} // namespace jas

// promotion with bf16 operands (the node element type of jasmine's expression trees is the
// std::common_type of its operands, mat_express_t.hpp:18-33): bf16 with bf16 or an integer
// stays bf16; with float or double it widens to that type
template <>
struct std::common_type<jas::bf16, jas::bf16> {
    using type = jas::bf16;
};
template <typename T>
requires std::is_arithmetic_v<T>
struct std::common_type<jas::bf16, T> {
    using type = std::conditional_t<std::is_floating_point_v<T>, std::common_type_t<float, T>, jas::bf16>;
};
template <typename T>
requires std::is_arithmetic_v<T>
struct std::common_type<T, jas::bf16> {
    using type = typename std::common_type<jas::bf16, T>::type;
};

#endif
