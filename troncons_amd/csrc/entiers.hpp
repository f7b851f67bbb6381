// entiers.hpp — integer helpers shared by the kernels and the host, free of HIP headers so that a
// plain C++ compiler can build them (the CPU tests compile this header with g++).
//
// - Diviseur: unsigned 32-bit division by a run-time invariant d as a multiply-high, a subtract
//   and two shifts (Granlund & Montgomery, "Division by Invariant Integers using Multiplication",
//   PLDI 1994, figure 4.1): l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1,
//   q = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0) with t = mulhi(m, n). Exact for every
//   n < 2^32 and 1 <= d <= 2^31. The slot decoders use it for a block's row (block / blocks per row).
// - elargir_u64: the 64-bit value whose halves two `readfirstlane` calls returned as int. Each half
//   goes through uint32_t before widening; widening the int itself would sign-extend a low word
//   with bit 31 set into the high word.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define TRC_HD __host__ __device__ __forceinline__
#else
#define TRC_HD inline
#endif

namespace trc {

TRC_HD uint32_t mulhi_u32(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __umulhi(a, b);
#else
    return uint32_t((uint64_t(a) * b) >> 32);
#endif
}

struct Diviseur {
    uint32_t d, m, s1, s2;

    TRC_HD static Diviseur de(uint32_t d) {
        Diviseur r;
        r.d = d;
        uint32_t l = 0;
        while (l < 32u && (uint64_t(1) << l) < d) ++l;  // ceil(log2 d)
        r.m = uint32_t(((uint64_t(1) << 32) * ((uint64_t(1) << l) - d)) / d + 1u);
        r.s1 = l < 1u ? l : 1u;
        r.s2 = l > 1u ? l - 1u : 0u;
        return r;
    }
    TRC_HD uint32_t quotient(uint32_t n) const {
        const uint32_t t = mulhi_u32(m, n);
        return (t + ((n - t) >> s1)) >> s2;
    }
};

TRC_HD uint64_t elargir_u64(int bas, int haut) {
    return uint64_t(uint32_t(bas)) | (uint64_t(uint32_t(haut)) << 32);
}

}  // namespace trc
