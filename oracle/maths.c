/*
 * maths.c — CPU restatement of the reference arithmetic on the hot path (TEST INFRASTRUCTURE, see
 * oracle.h): MXFP4 dequant, the GEMV in the reference's exact f32 operation order, its f64
 * reference, the router GEMV, SwiGLU, the ordered combine and the top-k router.
 *
 * Built with -ffp-contract=off: every a*b+c below is two roundings unless written fmaf().
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* gemv.cuh:26-29: 2^(e-128) in f32, exact for e = 0..255 (e = 0, 1 subnormal). */
float orc_echelle_e8m0(uint32_t e) {
    const uint32_t bits = e >= 2u ? (e - 1u) << 23 : (0x00200000u << e);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* gemv.cuh:33-36: doubled E2M1 magnitude from 0xC8643210, bit 3 = sign. */
float orc_valeur_e2m1x2(uint32_t c) {
    const float g = (float)((0xC8643210u >> ((c & 7u) << 2)) & 15u);
    return (c & 8u) ? -g : g;
}

static uint64_t al256(uint64_t x) { return (x + 255) & ~(uint64_t)255; }

/* produit_bloc, gemv.cuh:60-76: fixed order (word t, byte k, low then high nibble). */
static float produit_bloc(const uint8_t* q, const float* xb) {
    float s = 0.0f;
    for (int t = 0; t < 4; ++t)
        for (int k = 0; k < 4; ++k) {
            const uint8_t o = q[4 * t + k];
            s = fmaf(orc_valeur_e2m1x2(o & 15u), xb[4 * t + k], s);
            s = fmaf(orc_valeur_e2m1x2(o >> 4), xb[16 + 4 * t + k], s);
        }
    return s;
}

/* 32-lane xor butterfly (somme_warp_f32, gemv.cuh:78-82), value seen by lane 0. */
static float papillon32(float* v) {
    for (int d = 16; d > 0; d >>= 1) {
        float n[32];
        for (int l = 0; l < 32; ++l) n[l] = v[l] + v[l ^ d];
        memcpy(v, n, sizeof(n));
    }
    return v[0];
}

/* gemv_4_lignes, gemv.cuh:90-126 (one row at a time: the rows are independent). */
void orc_gemv_mxfp4(const uint8_t* mat, const float* x, float* y, uint32_t R, uint32_t C) {
    const uint32_t B = C / 32u;
    const uint64_t nb = (uint64_t)R * B;
    const uint8_t* ech = mat + al256(nb * 16);
    const uint8_t* biais = mat + al256(al256(nb * 16) + nb);
    for (uint32_t r = 0; r < R; ++r) {
        float acc[32];
        for (uint32_t l = 0; l < 32; ++l) {
            float a = 0.0f;
            for (uint32_t b = l; b < B; b += 32u) {
                const uint64_t beta = (uint64_t)r * B + b;
                a = fmaf(orc_echelle_e8m0(ech[beta]), produit_bloc(mat + 16 * beta, x + 32 * b), a);
            }
            acc[l] = a;
        }
        float bb;
        memcpy(&bb, biais + 4ull * r, 4);
        y[r] = papillon32(acc) + bb;
    }
}

/* f64 reference (banc_k.cu:1047-1072, tests/carte.rs:374-406): exact products, f64 sum. */
void orc_gemv_mxfp4_f64(const uint8_t* mat, const float* x, double* y, uint32_t R, uint32_t C) {
    const uint32_t B = C / 32u;
    const uint64_t nb = (uint64_t)R * B;
    const uint8_t* ech = mat + al256(nb * 16);
    const uint8_t* biais = mat + al256(al256(nb * 16) + nb);
    for (uint32_t r = 0; r < R; ++r) {
        double s = 0.0;
        for (uint32_t b = 0; b < B; ++b) {
            const uint64_t beta = (uint64_t)r * B + b;
            const double sc = ldexp(1.0, (int)ech[beta] - 128);
            for (int t = 0; t < 16; ++t) {
                const uint8_t q = mat[16 * beta + t];
                s += (double)orc_valeur_e2m1x2(q & 15u) * sc * (double)x[32 * b + t];
                s += (double)orc_valeur_e2m1x2(q >> 4) * sc * (double)x[32 * b + 16 + t];
            }
        }
        float bb;
        memcpy(&bb, biais + 4ull * r, 4);
        y[r] = s + (double)bb;
    }
}

/* gemv_f32_4_lignes, passe.cuh:104-130: lane l takes quads c = l, l+32, ...; x, y, z, w order. */
void orc_gemv_f32(const float* W, const float* x, const float* biais, float* y, uint32_t R, uint32_t C) {
    const uint32_t C4 = C / 4u;
    for (uint32_t r = 0; r < R; ++r) {
        float acc[32];
        for (uint32_t l = 0; l < 32; ++l) {
            float a = 0.0f;
            for (uint32_t c = l; c < C4; c += 32u) {
                const float* w = W + (uint64_t)r * C + 4ull * c;
                const float* xv = x + 4ull * c;
                a = fmaf(w[0], xv[0], a);
                a = fmaf(w[1], xv[1], a);
                a = fmaf(w[2], xv[2], a);
                a = fmaf(w[3], xv[3], a);
            }
            acc[l] = a;
        }
        const float s = papillon32(acc);
        y[r] = biais ? s + biais[r] : s;
    }
}

/* swiglu_oai, passe.cuh:598-605 / trc-reference ops.rs:133-140 */
void orc_swiglu_oai(const float* g, const float* u, float* y, uint32_t n) {
    for (uint32_t i = 0; i < n; ++i) {
        const double gv = fmin((double)g[i], 7.0);
        const double uv = fmin(fmax((double)u[i], -7.0), 7.0);
        y[i] = (float)(gv / (1.0 + exp(-1.702 * gv)) * (uv + 1.0));
    }
}

/* combiner, passe.cuh:611-622: each product and each sum rounded separately (no FMA). */
void orc_combiner(float* residu, const float* sorties, uint32_t pas, const float* poids, uint32_t n, uint32_t d) {
    for (uint32_t i = 0; i < d; ++i) {
        volatile float s = poids ? poids[0] * sorties[i] : sorties[i];
        for (uint32_t j = 1; j < n; ++j) {
            const float sj = sorties[(uint64_t)j * pas + i];
            volatile float p = poids ? poids[j] * sj : sj;
            s = s + p;
        }
        residu[i] = residu[i] + s;
    }
}

/* routeur_topk, passe.cuh:455-514 (selection: value desc, index asc; softmax of the k in f64). */
static int meilleur(float va, uint32_t ia, float vb, uint32_t ib) { return va > vb || (va == vb && ia < ib); }

void orc_routeur_topk(const float* logits, uint32_t E, uint32_t k, uint32_t* indices, float* poids) {
    unsigned char* pris = (unsigned char*)calloc(E, 1);
    float v[8];
    uint32_t idx[8];
    for (uint32_t r = 0; r < k; ++r) {
        float bv = -INFINITY;
        uint32_t bi = 0xFFFFFFFFu;
        for (uint32_t e = 0; e < E; ++e)
            if (!pris[e] && meilleur(logits[e], e, bv, bi)) {
                bv = logits[e];
                bi = e;
            }
        if (bi != 0xFFFFFFFFu) pris[bi] = 1;
        v[r] = bv;
        idx[r] = bi;
    }
    double ex[8], z = 0.0;
    const double m = v[0];
    for (uint32_t r = 0; r < k; ++r) {
        ex[r] = exp((double)v[r] - m);
        z += ex[r];
    }
    for (uint32_t r = 0; r < k; ++r) {
        indices[r] = idx[r];
        poids[r] = (float)(ex[r] / z);
    }
    free(pris);
}

/* routeur_topk_biais, passe.cuh:516-580 (the cache-biased router): the k are chosen on the f32
 * score logit + biais (score desc, index asc), then returned by unbiased logit desc, index asc
 * (insertion sort), weights = f64 softmax of the unbiased logits, max = the first. A slot left
 * unchosen (NaN scores) keeps index 0xFFFFFFFF and reads as logit -inf. */
void orc_routeur_topk_biais(const float* logits, const float* biais, uint32_t E, uint32_t k, uint32_t* indices,
                            float* poids) {
    unsigned char* pris = (unsigned char*)calloc(E, 1);
    uint32_t idx[8];
    float u[8];
    for (uint32_t r = 0; r < k; ++r) {
        float bv = -INFINITY;
        uint32_t bi = 0xFFFFFFFFu;
        for (uint32_t e = 0; e < E; ++e) {
            const volatile float sc = logits[e] + biais[e];
            if (!pris[e] && meilleur(sc, e, bv, bi)) {
                bv = sc;
                bi = e;
            }
        }
        if (bi != 0xFFFFFFFFu) pris[bi] = 1;
        idx[r] = bi;
        u[r] = bi < E ? logits[bi] : -INFINITY;
    }
    for (uint32_t r = 1; r < k; ++r)
        for (uint32_t j = r; j > 0 && meilleur(u[j], idx[j], u[j - 1], idx[j - 1]); --j) {
            const float tv = u[j];
            u[j] = u[j - 1];
            u[j - 1] = tv;
            const uint32_t ti = idx[j];
            idx[j] = idx[j - 1];
            idx[j - 1] = ti;
        }
    double ex[8], z = 0.0;
    const double m = u[0];
    for (uint32_t r = 0; r < k; ++r) {
        ex[r] = exp((double)u[r] - m);
        z += ex[r];
    }
    for (uint32_t r = 0; r < k; ++r) {
        indices[r] = idx[r];
        poids[r] = (float)(ex[r] / z);
    }
    free(pris);
}
