// va_keys.hpp — 32-bit ordering keys of the top-k paths (host and device; no HIP dependency, so
// host-only test programs can include it).
#pragma once

#include <cstdint>

#ifdef __HIPCC__
#define VA_HD __host__ __device__
#else
#define VA_HD
#endif

namespace va {

// 0xFFFFFFFF is the key of an absent item (a row excluded from a search, e.g. a deleted row of
// an index): selections order it after every real key and output it as a missing result.
constexpr uint32_t kAbsentKey = 0xFFFFFFFFu;
// Ascending-orderable key of a float: -0 and +0 map to one key, NaN to the largest real key
// (0xFFFFFFFE, after +inf).
VA_HD inline uint32_t key_of_float(float f) {
    if (f != f) return 0xFFFFFFFEu;
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if (f == 0.0f) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
VA_HD inline float float_of_key(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
    return __builtin_bit_cast(float, u);
}
// Descending order (MAX mode), NaN still last.
VA_HD inline uint32_t key_of_float_desc(float f) {
    if (f != f) return 0xFFFFFFFEu;
    return ~key_of_float(f);
}
VA_HD inline float float_of_key_desc(uint32_t k) { return float_of_key(~k); }
// int32 ascending key
VA_HD inline uint32_t key_of_i32(int32_t v) { return uint32_t(v) ^ 0x80000000u; }
VA_HD inline int32_t i32_of_key(uint32_t k) { return int32_t(k ^ 0x80000000u); }

}  // namespace va
