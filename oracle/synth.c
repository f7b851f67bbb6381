/*
 * synth.c — seeded generators and the synthetic workload definition (TEST INFRASTRUCTURE, see
 * oracle.h), plus bf16 conversion and empreinte64 (SHA-256 prefix).
 *
 * splitmix64 follows moteur/crates/trc-noyaux/tests/carte.rs:22-31; xorshift64* follows
 * moteur/crates/trc-codec/tests/rans.rs:20-27. The synthetic MXFP4 workload itself is this
 * build's definition (the BASELINE configs describe it in words); the product's generator
 * (troncons_amd/csrc/codeur.cpp) restates the same definition and tests compare the two.
 */
#include <math.h>
#include <string.h>

#include "oracle.h"

uint64_t orc_splitmix64(uint64_t* etat) {
    *etat += 0x9E3779B97F4A7C15ull;
    uint64_t z = *etat;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t orc_xorshift64s(uint64_t* etat) {
    *etat ^= *etat >> 12;
    *etat ^= *etat << 25;
    *etat ^= *etat >> 27;
    return *etat * 0x2545F4914F6CDD1Dull;
}

uint16_t orc_bf16_depuis_f32(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x7FFFFFu)) return (uint16_t)((b >> 16) | 0x40);
    const uint32_t arrondi = 0x7FFFu + ((b >> 16) & 1u);
    return (uint16_t)((b + arrondi) >> 16);
}

float orc_f32_depuis_bf16(uint16_t h) {
    const uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* Key of a generator stream: (seed, layer, expert, slot). */
static uint64_t etat_initial(uint64_t graine, uint32_t couche, uint32_t expert, uint32_t cle) {
    const uint64_t k = ((uint64_t)(couche & 0xFFFFFFu) << 40) ^ ((uint64_t)(expert & 0xFFFFFFu) << 16) ^ (uint64_t)(cle & 0xFFFFu);
    return graine ^ (k * 0xD1B54A32D192ED03ull);
}

/* Nibble law "A": p(code) over the 16 E2M1 codes, symmetric; zero carries a random sign
 * (p(+0) = p(-0) = 0.10) so that the v1.2 encoder's -0 -> +0 fold gives p(0) = 0.20. */
static const double PMF_A[16] = {0.10, 0.14, 0.13, 0.06, 0.035, 0.02, 0.01, 0.005,
                                 0.10, 0.14, 0.13, 0.06, 0.035, 0.02, 0.01, 0.005};

static uint32_t tirer_demi(uint64_t* etat, const double* cdf) {
    const double u = (double)(orc_splitmix64(etat) >> 11) * 0x1.0p-53;
    for (uint32_t c = 0; c < 15; ++c)
        if (u < cdf[c]) return c;
    return 15;
}

static void normales(uint64_t* etat, uint32_t n, float sigma, float* out) {
    for (uint32_t i = 0; i < n; i += 2) {
        const double u1 = (double)((orc_splitmix64(etat) >> 11) + 1) * 0x1.0p-53;
        const double u2 = (double)(orc_splitmix64(etat) >> 11) * 0x1.0p-53;
        const double r = sqrt(-2.0 * log(u1));
        const double a = 6.283185307179586 * u2;
        const float z0 = (float)((double)sigma * (r * cos(a)));
        const float z1 = (float)((double)sigma * (r * sin(a)));
        out[i] = orc_f32_depuis_bf16(orc_bf16_depuis_f32(z0));
        if (i + 1 < n) out[i + 1] = orc_f32_depuis_bf16(orc_bf16_depuis_f32(z1));
    }
}

void orc_synth_matrice(uint64_t graine, uint32_t couche, uint32_t expert, uint32_t cle, uint32_t R, uint32_t C,
                       uint8_t* blocs17, float* biais) {
    uint64_t etat = etat_initial(graine, couche, expert, cle);
    const uint64_t nb = (uint64_t)R * (C / 32);
    double cdf[16], acc = 0.0;
    for (int c = 0; c < 16; ++c) {
        acc += PMF_A[c];
        cdf[c] = acc;
    }
    /* 1. E8M0 scales, uniform in [119, 125] (2^-8 .. 2^-2 in the 2^(e-127) convention) */
    for (uint64_t b = 0; b < nb; ++b) blocs17[17 * b] = (uint8_t)(119 + orc_splitmix64(&etat) % 7);
    /* 2. the 16 code bytes of each block: low nibble drawn first, then high */
    for (uint64_t b = 0; b < nb; ++b)
        for (int i = 0; i < 16; ++i) {
            const uint32_t lo = tirer_demi(&etat, cdf);
            const uint32_t hi = tirer_demi(&etat, cdf);
            blocs17[17 * b + 1 + i] = (uint8_t)(lo | (hi << 4));
        }
    /* 3. biases: bf16 N(0, 0.02) */
    if (biais) normales(&etat, R, 0.02f, biais);
}

void orc_synth_normale_bf16(uint64_t graine, uint32_t cle1, uint32_t cle2, uint32_t n, float sigma, float* out) {
    uint64_t etat = etat_initial(graine, cle1, 0xFFFFFFu, cle2);
    normales(&etat, n, sigma, out);
}

/* ---- SHA-256 (FIPS 180-4) for empreinte64, trc-format/src/lib.rs:111-116 ------------------------ */
static const uint32_t K256[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

static uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static void sha_bloc(uint32_t* h, const uint8_t* p) {
    uint32_t w[64];
    for (int i = 0; i < 16; ++i) w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 | (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
    for (int i = 16; i < 64; ++i) {
        const uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
        const uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; ++i) {
        const uint32_t t1 = hh + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) + K256[i] + w[i];
        const uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
        hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}

uint64_t orc_empreinte64(const uint8_t* o, size_t n) {
    uint32_t h[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a, 0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    size_t i = 0;
    for (; i + 64 <= n; i += 64) sha_bloc(h, o + i);
    uint8_t fin[128];
    memset(fin, 0, sizeof(fin));
    const size_t reste = n - i;
    memcpy(fin, o + i, reste);
    fin[reste] = 0x80;
    const size_t nfin = reste + 9 <= 64 ? 64 : 128;
    const uint64_t bits = (uint64_t)n * 8;
    for (int k = 0; k < 8; ++k) fin[nfin - 1 - k] = (uint8_t)(bits >> (8 * k));
    sha_bloc(h, fin);
    if (nfin == 128) sha_bloc(h, fin + 64);
    /* first 8 digest bytes (big-endian words h0, h1) read as a little-endian u64 */
    uint8_t d[8];
    for (int k = 0; k < 4; ++k) {
        d[k] = (uint8_t)(h[0] >> (24 - 8 * k));
        d[4 + k] = (uint8_t)(h[1] >> (24 - 8 * k));
    }
    uint64_t v = 0;
    for (int k = 7; k >= 0; --k) v = (v << 8) | d[k];
    return v;
}
