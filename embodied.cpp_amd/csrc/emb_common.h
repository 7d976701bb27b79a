// Internal helpers shared by the host and HIP sources of libemb_kv.so.
#pragma once

#include <cstdint>
#include <cstdio>
#include <string>

#include "emb_kv.h"

namespace emb {

// Records a message for emb_last_error() (thread-local) and returns code.
int set_error(int code, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

#if defined(__HIP__)  // device helpers, for the .hip sources
// Element offset, inside one f16 V-shadow page of one kv head, of dim d and
// page row t: the 16 keys of a dim sit in the order the attention P.V MFMA
// reads them (row t at position P = t with bits 2 and 3 swapped), the two
// 8-key halves exchanged when bit 3 of d is set (LDS bank spread).
__host__ __device__ inline int v16_index(int d, int t) {
    const int P = (t & 3) | ((t >> 1) & 4) | ((t << 1) & 8);
    return d * 16 + (((P >> 3) ^ ((d >> 3) & 1)) << 3) + (P & 7);
}
#endif

// std::mt19937_64-compatible engine (same constants as the C++ standard).
struct Mt64 {
    uint64_t mt[312];
    int idx = 312;
    explicit Mt64(uint64_t seed) {
        mt[0] = seed;
        for (int i = 1; i < 312; ++i) mt[i] = 6364136223846793005ULL * (mt[i - 1] ^ (mt[i - 1] >> 62)) + (uint64_t)i;
    }
    uint64_t next() {
        if (idx >= 312) {
            for (int i = 0; i < 312; ++i) {
                uint64_t x = (mt[i] & 0xFFFFFFFF80000000ULL) | (mt[(i + 1) % 312] & 0x7FFFFFFFULL);
                uint64_t xa = (x >> 1) ^ ((x & 1ULL) ? 0xB5026F5AA96619E9ULL : 0ULL);
                mt[i] = mt[(i + 156) % 312] ^ xa;
            }
            idx = 0;
        }
        uint64_t x = mt[idx++];
        x ^= (x >> 29) & 0x5555555555555555ULL;
        x ^= (x << 17) & 0x71D67FFFEDA60000ULL;
        x ^= (x << 37) & 0xFFF7EEE000000000ULL;
        x ^= x >> 43;
        return x;
    }
};

}  // namespace emb

#define EMB_CHECK_ARG(cond, ...)                                  \
    do {                                                          \
        if (!(cond)) return emb::set_error(EMB_ERR_ARG, __VA_ARGS__); \
    } while (0)
