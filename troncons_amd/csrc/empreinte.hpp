// empreinte.hpp — SHA-256 (FIPS 180-4) and the .trc fingerprint empreinte64 (the first 8 bytes of
// SHA-256, read as a little-endian u64; ARCHITECTURE.md §4.12, trc-format/src/lib.rs:111-127).
//
// The round constants and the initial hash are derived at start-up from their definition (the
// first 32 bits of the fractional parts of the cube roots of the first 64 primes, and of the square
// roots of the first 8), not typed in.
#pragma once

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>

namespace trc {

class Sha256 {
public:
    Sha256() { remettre(); }

    void remettre() {
        const Constantes& k = constantes();
        std::memcpy(h_, k.h0, sizeof(h_));
        n_ = 0;
        pris_ = 0;
    }

    void ajouter(const uint8_t* p, size_t n) {
        n_ += n;
        if (pris_) {
            const size_t k = n < 64 - pris_ ? n : 64 - pris_;
            std::memcpy(tampon_ + pris_, p, k);
            pris_ += k;
            p += k;
            n -= k;
            if (pris_ < 64) return;
            bloc(tampon_);
            pris_ = 0;
        }
        for (; n >= 64; p += 64, n -= 64) bloc(p);
        std::memcpy(tampon_, p, n);
        pris_ = n;
    }

    void finir(uint8_t sortie[32]) {
        const uint64_t bits = n_ * 8u;
        const uint8_t un = 0x80;
        ajouter(&un, 1);
        const uint8_t zero[64] = {0};
        ajouter(zero, (pris_ <= 56) ? 56 - pris_ : 120 - pris_);
        uint8_t lg[8];
        for (int i = 0; i < 8; ++i) lg[i] = uint8_t(bits >> (56 - 8 * i));
        ajouter(lg, 8);
        for (int i = 0; i < 8; ++i)
            for (int j = 0; j < 4; ++j) sortie[4 * i + j] = uint8_t(h_[i] >> (24 - 8 * j));
    }

private:
    struct Constantes {
        uint32_t k[64];
        uint32_t h0[8];
        Constantes() {
            int premiers[64];
            int n = 0;
            for (int c = 2; n < 64; ++c) {
                bool p = true;
                for (int d = 2; d * d <= c; ++d)
                    if (c % d == 0) {
                        p = false;
                        break;
                    }
                if (p) premiers[n++] = c;
            }
            for (int i = 0; i < 64; ++i) k[i] = fraction32(std::cbrt((long double)premiers[i]));
            for (int i = 0; i < 8; ++i) h0[i] = fraction32(std::sqrt((long double)premiers[i]));
        }
        static uint32_t fraction32(long double x) {
            const long double f = x - std::floor(x);
            return uint32_t(std::floor(std::ldexp(f, 32)));
        }
    };
    static const Constantes& constantes() {
        static const Constantes c;
        return c;
    }
    static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

    void bloc(const uint8_t* p) {
        const uint32_t* K = constantes().k;
        uint32_t w[64];
        for (int i = 0; i < 16; ++i)
            w[i] = (uint32_t(p[4 * i]) << 24) | (uint32_t(p[4 * i + 1]) << 16) | (uint32_t(p[4 * i + 2]) << 8) |
                   uint32_t(p[4 * i + 3]);
        for (int i = 16; i < 64; ++i) {
            const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
            const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
            w[i] = w[i - 16] + s0 + w[i - 7] + s1;
        }
        uint32_t a = h_[0], b = h_[1], c = h_[2], d = h_[3], e = h_[4], f = h_[5], g = h_[6], h = h_[7];
        for (int i = 0; i < 64; ++i) {
            const uint32_t S1 = rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25);
            const uint32_t ch = (e & f) ^ (~e & g);
            const uint32_t t1 = h + S1 + ch + K[i] + w[i];
            const uint32_t S0 = rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22);
            const uint32_t maj = (a & b) ^ (a & c) ^ (b & c);
            const uint32_t t2 = S0 + maj;
            h = g;
            g = f;
            f = e;
            e = d + t1;
            d = c;
            c = b;
            b = a;
            a = t1 + t2;
        }
        h_[0] += a;
        h_[1] += b;
        h_[2] += c;
        h_[3] += d;
        h_[4] += e;
        h_[5] += f;
        h_[6] += g;
        h_[7] += h;
    }

    uint32_t h_[8];
    uint64_t n_;
    uint8_t tampon_[64];
    size_t pris_;
};

inline uint64_t empreinte64_de(const uint8_t (&d)[32]) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; --i) v = (v << 8) | d[i];
    return v;
}

inline uint64_t empreinte64(const uint8_t* p, size_t n) {
    Sha256 s;
    s.ajouter(p, n);
    uint8_t d[32];
    s.finir(d);
    return empreinte64_de(d);
}

}  // namespace trc
