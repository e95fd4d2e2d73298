// Internal helpers shared by the host sources of libqwenny_hip: error reporting across the C ABI and small
// conversions.
#pragma once
#include <stdint.h>
#include <string.h>

#include <cstdio>
#include <string>

#include "../../include/qwenny_hip.h"

namespace qh {

// Record `msg` as the calling thread's last error and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// f32 -> bf16 bits, round to nearest even (NaN kept quiet).
inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

inline float bf16_to_f32(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

// Run fn(lo, hi) over [0, n) split across the host's threads.
void parallel_for(size_t n, void (*fn)(void*, size_t, size_t), void* arg);

template <class F>
void parallel(size_t n, F&& f) {
    parallel_for(
        n, [](void* a, size_t lo, size_t hi) { (*static_cast<F*>(a))(lo, hi); }, &f);
}

}  // namespace qh
