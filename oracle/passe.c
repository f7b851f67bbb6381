/*
 * passe.c — CPU restatement of the reference's forward-pass operations around the expert path
 * (TEST INFRASTRUCTURE, see oracle.h): Q8_0 GEMV and row, RMSNorm, YaRN rotation, the f16 KV
 * cache write, decode attention with per-head sinks, argmax. Each follows the operation order of
 * the reference kernel it cites (moteur/crates/trc-noyaux/noyaux/passe.cuh), so that a kernel
 * following the same order can be compared bit for bit where the reference is exact.
 *
 * Built with -ffp-contract=off: every a*b+c below is two roundings unless written fmaf()/fma().
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* f16 bits -> f32, exact (passe.cuh:43-45). */
float orc_f32_depuis_f16(uint16_t h) {
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 31u)
        bits = s | 0x7F800000u | (m << 13);
    else if (e != 0u)
        bits = s | ((e + 112u) << 23) | (m << 13);
    else if (m == 0u)
        bits = s;
    else {  /* subnormal: m * 2^-24, renormalised */
        uint32_t k = 0;
        while (!(m & 0x400u)) {
            m <<= 1;
            ++k;
        }
        bits = s | ((113u - k) << 23) | ((m & 0x3FFu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* f32 -> f16 bits, round to nearest, ties to even (__float2half_rn, passe.cuh:294-295):
 * overflow to infinity, f16 subnormals kept, NaN kept quiet. */
uint16_t orc_f16_depuis_f32(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint16_t s = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t e = (x >> 23) & 0xFFu, m = x & 0x7FFFFFu;
    if (e == 0xFFu) return (uint16_t)(s | 0x7C00u | (m ? 0x200u | (m >> 13) : 0u));
    if (e == 0u) return s; /* f32 zero or subnormal: below half of the smallest f16 subnormal */
    const uint32_t mant = m | 0x800000u;  /* value = mant * 2^(e - 150) */
    const int32_t E = (int32_t)e - 112;   /* f16 exponent field if normal */
    uint32_t decal = E >= 1 ? 13u : (uint32_t)(13 + 1 - E);
    if (decal > 24u) return s;
    uint32_t q = mant >> decal;
    const uint32_t reste = mant & ((1u << decal) - 1u), moitie = 1u << (decal - 1u);
    if (reste > moitie || (reste == moitie && (q & 1u))) ++q;
    if (E >= 1) {
        /* q in [0x400, 0x800]: 0x800 carries into the exponent */
        uint32_t champ = (uint32_t)E;
        if (q == 0x800u) {
            q = 0x400u;
            ++champ;
        }
        if (champ >= 31u) return (uint16_t)(s | 0x7C00u);
        return (uint16_t)(s | (champ << 10) | (q & 0x3FFu));
    }
    /* subnormal result: q in [0, 0x400]; 0x400 is the smallest normal, encoded as such */
    return (uint16_t)(s | q);
}

static float papillon32(float* v) {
    for (int d = 16; d > 0; d >>= 1) {
        float n[32];
        for (int l = 0; l < 32; ++l) n[l] = v[l] + v[l ^ d];
        memcpy(v, n, sizeof(n));
    }
    return v[0];
}

/* gemv_q8_0_4_lignes, passe.cuh:52-97: lane l takes blocks b = l, l + 32, ...; in a block
 * s = sum over i of q_i x_i (one fmaf chain, words t = 0..15, low byte then high byte), then
 * acc = fmaf(d, s, acc); butterfly over the 32 lanes; + bias. */
void orc_gemv_q8_0(const uint8_t* W, const float* x, const float* biais, float* y, uint32_t R, uint32_t C) {
    const uint32_t B = C / 32u;
    for (uint32_t r = 0; r < R; ++r) {
        float acc[32];
        for (uint32_t l = 0; l < 32; ++l) {
            float a = 0.0f;
            for (uint32_t b = l; b < B; b += 32u) {
                const uint8_t* blk = W + ((uint64_t)r * B + b) * 34u;
                const float d = orc_f32_depuis_f16((uint16_t)(blk[0] | (blk[1] << 8)));
                float s = 0.0f;
                for (uint32_t t = 0; t < 16; ++t) {
                    s = fmaf((float)(int8_t)blk[2 + 2 * t], x[32 * b + 2 * t], s);
                    s = fmaf((float)(int8_t)blk[3 + 2 * t], x[32 * b + 2 * t + 1], s);
                }
                a = fmaf(d, s, a);
            }
            acc[l] = a;
        }
        const float s = papillon32(acc);
        y[r] = biais ? s + biais[r] : s;
    }
}

/* ligne_q8_0, passe.cuh:627-637: y[i] = d * q_i (exact). */
void orc_ligne_q8_0(const uint8_t* W, uint32_t ligne, uint32_t C, float* y) {
    const uint32_t B = C / 32u;
    for (uint32_t i = 0; i < C; ++i) {
        const uint8_t* blk = W + ((uint64_t)ligne * B + i / 32u) * 34u;
        const float d = orc_f32_depuis_f16((uint16_t)(blk[0] | (blk[1] << 8)));
        y[i] = d * (float)(int8_t)blk[2 + (i & 31u)];
    }
}

/* rmsnorm, passe.cuh:235-259: per row, thread t of 256 sums x_i^2 for i = t, t + 256, ... with f64
 * fma, fixed tree over the 256 partial sums, r = 1/sqrt(sum/n + eps), y_i = (x_i * r) * w_i in f64,
 * rounded once. */
void orc_rmsnorm(const float* x, const float* w, float* y, uint32_t n, uint32_t lignes, float eps) {
    for (uint32_t l = 0; l < lignes; ++l) {
        const float* xr = x + (uint64_t)l * n;
        float* yr = y + (uint64_t)l * n;
        double part[256];
        for (uint32_t t = 0; t < 256; ++t) {
            double s = 0.0;
            for (uint32_t i = t; i < n; i += 256u) s = fma((double)xr[i], (double)xr[i], s);
            part[t] = s;
        }
        for (uint32_t k = 128; k > 0; k >>= 1)
            for (uint32_t t = 0; t < k; ++t) part[t] += part[t + k];
        const double r = 1.0 / sqrt(part[0] / (double)n + (double)eps);
        for (uint32_t i = 0; i < n; ++i) yr[i] = (float)((double)xr[i] * r * (double)w[i]);
    }
}

/* inv_freq_yarn, passe.cuh:145-167 (trc-reference ops.rs:46-70): inv_freq of pair i and the
 * concentration 0.1 ln(s) + 1, in f64; bas/haut: the ramp bounds (rounded for variant 1). */
double orc_inv_freq_yarn(const orc_params_rope* p, uint32_t i, double* concentration, double* bas_out,
                         double* haut_out) {
    const uint32_t demi = p->dim_tete / 2u;
    const double freq = pow(p->base, (double)(2u * i) / (double)p->dim_tete);
    if (p->facteur <= 1.0) {
        *concentration = 1.0;
        if (bas_out) *bas_out = 0.0;
        if (haut_out) *haut_out = 0.0;
        return 1.0 / freq;
    }
    *concentration = 0.1 * log(p->facteur) + 1.0;
    const double deux_pi = 6.283185307179586476925286766559;
    double bas = (double)demi * log(p->ctx_origine / (p->beta_rapide * deux_pi)) / log(p->base);
    double haut = (double)demi * log(p->ctx_origine / (p->beta_lent * deux_pi)) / log(p->base);
    if (p->variante == 1u) {
        bas = fmax(floor(bas), 0.0);
        haut = fmin(ceil(haut), (double)(p->dim_tete - 1u));
    }
    if (bas_out) *bas_out = bas;
    if (haut_out) *haut_out = haut;
    const double interpolation = 1.0 / (p->facteur * freq);
    const double extrapolation = 1.0 / freq;
    const double rampe = fmin(fmax(((double)i - bas) / (haut - bas), 0.0), 1.0);
    const double masque = 1.0 - rampe;
    return interpolation * (1.0 - masque) + extrapolation * masque;
}

/* rope_yarn, passe.cuh:261-284: NEOX half rotation of every head of q then k, in place, in f64:
 * o1 = x1 c - x2 s, o2 = x2 c + x1 s with c, s the cosine and sine of position * inv_freq, each
 * times the concentration. */
void orc_rope_yarn(float* q, float* k, uint32_t tetes_q, uint32_t tetes_k, uint32_t position,
                   const orc_params_rope* p) {
    const uint32_t d = p->dim_tete, demi = d / 2u;
    for (uint32_t h = 0; h < tetes_q + tetes_k; ++h) {
        float* x = h < tetes_q ? q + (uint64_t)h * d : k + (uint64_t)(h - tetes_q) * d;
        for (uint32_t i = 0; i < demi; ++i) {
            double m;
            const double inv = orc_inv_freq_yarn(p, i, &m, NULL, NULL);
            double s = sin((double)position * inv), c = cos((double)position * inv);
            c *= m;
            s *= m;
            const double a = x[i], b = x[i + demi];
            x[i] = (float)(a * c - b * s);
            x[i + demi] = (float)(b * c + a * s);
        }
    }
}

/* ecrire_kv, passe.cuh:286-296: k and v rounded to f16 into slot case_kv ([slot][dkv]). */
void orc_ecrire_kv(const float* k, const float* v, uint16_t* cache_k, uint16_t* cache_v, uint32_t dkv,
                   uint32_t case_kv) {
    for (uint32_t i = 0; i < dkv; ++i) {
        cache_k[(uint64_t)case_kv * dkv + i] = orc_f16_depuis_f32(k[i]);
        cache_v[(uint64_t)case_kv * dkv + i] = orc_f16_depuis_f32(v[i]);
    }
}

/* attention, passe.cuh:298-373, one query head at a time (heads are independent): scores in f32
 * (fmaf chain over d = 0..63, then times the scale); m = max(max_j score, sink); e_j = expf(score
 * - m); z = fixed tree over the 256 threads' sums (thread t adds j = t, t + 256, ... in order) +
 * expf(sink - m); out[t] = ((G0 + G1) + (G2 + G3)) / z with G_g the fmaf chain over j = g, g + 4,
 * ... of e_j v_j[t]. Head h reads kv head h / (heads / kv heads); position pos is in slot pos,
 * or pos mod anneau. */
void orc_attention(const float* q, const uint16_t* cache_k, const uint16_t* cache_v, const float* puits,
                   float* sortie, const orc_params_attention* p) {
    const uint32_t D = 64, n = p->fin - p->debut, dkv = p->tetes_kv * D;
    float* e = (float*)malloc(sizeof(float) * (n ? n : 1));
    for (uint32_t h = 0; h < p->tetes; ++h) {
        const uint32_t hk = h / (p->tetes / p->tetes_kv);
        const float* qs = q + (uint64_t)h * D;
        float m = -INFINITY;
        for (uint32_t j = 0; j < n; ++j) {
            const uint32_t pos = p->debut + j, c = p->anneau ? pos % p->anneau : pos;
            const uint16_t* kr = cache_k + (uint64_t)c * dkv + (uint64_t)hk * D;
            float s = 0.0f;
            for (uint32_t t = 0; t < D; ++t) s = fmaf(qs[t], orc_f32_depuis_f16(kr[t]), s);
            e[j] = s * p->echelle;
            m = fmaxf(m, e[j]);
        }
        m = fmaxf(m, puits[h]);
        float part[256];
        for (uint32_t t = 0; t < 256; ++t) part[t] = 0.0f;
        for (uint32_t j = 0; j < n; ++j) {
            e[j] = expf(e[j] - m);
            part[j % 256u] += e[j];
        }
        for (uint32_t k = 128; k > 0; k >>= 1)
            for (uint32_t t = 0; t < k; ++t) part[t] = part[t] + part[t + k];
        const float z = part[0] + expf(puits[h] - m);
        for (uint32_t t = 0; t < D; ++t) {
            float g[4];
            for (uint32_t gg = 0; gg < 4; ++gg) {
                float a = 0.0f;
                for (uint32_t j = gg; j < n; j += 4u) {
                    const uint32_t pos = p->debut + j, c = p->anneau ? pos % p->anneau : pos;
                    a = fmaf(e[j], orc_f32_depuis_f16(cache_v[(uint64_t)c * dkv + (uint64_t)hk * D + t]), a);
                }
                g[gg] = a;
            }
            sortie[(uint64_t)h * D + t] = ((g[0] + g[1]) + (g[2] + g[3])) / z;
        }
    }
    free(e);
}

/* argmax, passe.cuh:639-666: largest value, ties to the lower index, NaN never chosen
 * (0xFFFFFFFF when every value is NaN). */
uint32_t orc_argmax(const float* v, uint32_t n) {
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t i = 0; i < n; ++i)
        if (v[i] > bv || (v[i] == bv && i < bi)) {
            bv = v[i];
            bi = i;
        }
    return bi;
}
