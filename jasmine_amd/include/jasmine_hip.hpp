// C++ side of the boundary: status codes -> the exception types jasmine throws, RAII device
// buffers, element-type -> jas_dtype mapping.  Included by every jasmine-API header.
#ifndef JASMINE_AMD_JASMINE_HIP_HPP
#define JASMINE_AMD_JASMINE_HIP_HPP

#include <atomic>
#include <cstdint>
#include <cstring>
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

template <typename T>
constexpr int dtype_of()
{
    if constexpr (std::is_same_v<T, float>) return JAS_F32;
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

#endif
