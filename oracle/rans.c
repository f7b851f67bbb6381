/*
 * rans.c — CPU restatement of the reference rANS codec (TEST INFRASTRUCTURE, see oracle.h).
 *
 * Follows moteur/crates/trc-codec/src/rans.rs (normative text: decisions/ARCHITECTURE.md:577-620).
 * Arithmetic is on uint32_t / uint64_t exactly where the reference uses u32 / u64; u32 products
 * wrap like the reference's release build and like the GPU kernels.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static inline uint32_t rd32(const uint8_t* p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }
static inline uint32_t rd16(const uint8_t* p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8; }
static inline void wr32(uint8_t* p, uint32_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); p[2] = (uint8_t)(v >> 16); p[3] = (uint8_t)(v >> 24); }
static inline void wr16(uint8_t* p, uint32_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

static int n_symboles(int g) { return g == 1 ? 256 : 16; }   /* rans.rs:48-54 */
static int sous_pas(int g) { return g == 1 ? 4 : 8; }         /* rans.rs:41-47 */

/* ---- TableRans::depuis_comptes, rans.rs:83-127 ---------------------------------------------- */
void orc_table_depuis_comptes(const uint64_t* c, int geometrie, uint16_t* freq_out) {
    const int n = n_symboles(geometrie);
    uint64_t comptes[256];
    uint64_t total = 0;
    for (int i = 0; i < n; ++i) {
        comptes[i] = c[i];
        total += c[i];
    }
    if (total == 0) { /* rans.rs:87-89: all-zero counts give symbol 0 the whole mass */
        comptes[0] = 1;
        total = 1;
    }
    int64_t freq[256];
    for (int i = 0; i < n; ++i) {
        freq[i] = 0;
        if (comptes[i] > 0) {
            /* rans.rs:94: ((c as f64) * (M as f64) / (total as f64)).round(); round() = half away
             * from zero, as C round(). */
            double v = round(((double)comptes[i] * (double)ORC_M) / (double)total);
            int64_t f = (int64_t)v;
            freq[i] = f < 1 ? 1 : f;
        }
    }
    int64_t somme = 0;
    for (int i = 0; i < n; ++i) somme += freq[i];
    int fait = 0;
    if (geometrie == 2) {
        /* rans.rs:100-107: Iterator::max_by_key returns the LAST maximal element */
        int imax = 0;
        for (int i = 0; i < n; ++i)
            if (freq[i] >= freq[imax]) imax = i;
        int64_t corrige = freq[imax] + ((int64_t)ORC_M - somme);
        if (corrige >= 1) {
            freq[imax] = corrige;
            fait = 1;
        }
    }
    if (!fait) {
        /* rans.rs:108-124: stable sort by decreasing frequency (ties: increasing index), then
         * walk it cyclically, one unit at a time, never below 1. */
        int ordre[256];
        for (int i = 0; i < n; ++i) ordre[i] = i;
        for (int i = 1; i < n; ++i) { /* insertion sort: stable */
            int v = ordre[i], k = i;
            while (k > 0 && freq[ordre[k - 1]] < freq[v]) {
                ordre[k] = ordre[k - 1];
                --k;
            }
            ordre[k] = v;
        }
        long j = 0;
        while (somme != (int64_t)ORC_M) {
            int i = ordre[j % n];
            if (somme > (int64_t)ORC_M && freq[i] > 1) {
                freq[i] -= 1;
                somme -= 1;
            } else if (somme < (int64_t)ORC_M && freq[i] > 0) {
                freq[i] += 1;
                somme += 1;
            }
            ++j;
        }
    }
    for (int i = 0; i < n; ++i) freq_out[i] = (uint16_t)freq[i];
}

/* ---- TableRans::construire / depuis_frequences, rans.rs:131-166 ------------------------------ */
int orc_lut(const uint16_t* freq, int geometrie, uint32_t* cumul_out, uint32_t* lut_out) {
    if (geometrie != 1 && geometrie != 2) return -1;
    const int n = n_symboles(geometrie);
    uint32_t somme = 0;
    for (int s = 0; s < n; ++s) {
        if (freq[s] > ORC_M) return -1;
        somme += freq[s];
    }
    if (somme != ORC_M) return -1;
    uint32_t c = 0;
    for (int s = 0; s < n; ++s) {
        const uint32_t f = freq[s];
        if (cumul_out) cumul_out[s] = c;
        for (uint32_t i = c; i < c + f; ++i) {
            if (geometrie == 1)
                lut_out[i] = (uint32_t)s | ((f - 1u) << 8) | ((i - c) << 20);
            else
                lut_out[i] = (uint32_t)s | (f << 4) | ((i - c) << 17);
        }
        c += f;
    }
    return 0;
}

/* ---- luts_couche, abi.rs:210-221 -------------------------------------------------------------- */
int orc_luts_couche(const uint16_t* const* freqs, uint32_t* luts_out) {
    memset(luts_out, 0, sizeof(uint32_t) * 3u * 4u * ORC_M);
    for (int j = 0; j < 3; ++j)
        for (int t = 0; t < 4; ++t)
            if (freqs[j * 4 + t] && orc_lut(freqs[j * 4 + t], 1, NULL, luts_out + (size_t)(j * 4 + t) * ORC_M) != 0)
                return -1;
    return 0;
}

/* ---- FluxRans::lire, rans.rs:231-280 ----------------------------------------------------------- */
int orc_flux_lire(const uint8_t* b, size_t len, orc_flux* out) {
    if (len < ORC_ENTETE_FLUX) return -1;
    const uint32_t P = rd32(b), N = rd16(b + 4), g = b[6];
    const uint64_t nt = rd32(b + 8), nw = rd32(b + 12);
    if (b[7] != 0) return -1;
    if (g != 1 && g != 2) return -1;
    if (P % ORC_OCTETS_PAR_MACRO != 0 || N == 0) return -1;
    const uint64_t macro = P / ORC_OCTETS_PAR_MACRO;
    if (nt != (macro + N - 1) / N) return -1;
    const uint64_t fin = ORC_ENTETE_FLUX + 4 * nt + 4 * ORC_VOIES * nt + 2 * nw;
    if (fin > len) return -1;
    for (size_t i = fin; i < len; ++i)
        if (b[i] != 0) return -1;
    const uint8_t* deb = b + ORC_ENTETE_FLUX;
    for (uint64_t t = 0; t < nt; ++t) {
        uint32_t d = rd32(deb + 4 * t);
        if (t == 0 && d != 0) return -1;
        if (t > 0 && rd32(deb + 4 * (t - 1)) > d) return -1;
        if (t + 1 == nt && d > nw) return -1;
    }
    out->P = P;
    out->N = N;
    out->geometrie = g;
    out->T = (uint32_t)nt;
    out->W = (uint32_t)nw;
    out->debuts = deb;
    out->etats = deb + 4 * nt;
    out->mots = deb + 4 * nt + 4 * ORC_VOIES * nt;
    return 0;
}

static inline int contexte(int g, const uint8_t* kappa, size_t n_kappa, size_t n) {
    if (g != 1 || kappa == NULL) return 0;
    size_t blk = n / 16; /* rans.rs:356-362: kappa[n/16], 0 beyond */
    return blk < n_kappa ? kappa[blk] : 0;
}

/* ---- coder_avec + serialiser, rans.rs:296-334, 208-227 ---------------------------------------- */
size_t orc_coder(const uint8_t* source, size_t P, int geometrie, const uint8_t* kappa, size_t n_kappa,
                 const uint16_t* freqs, int ntables, uint32_t N, uint8_t* out, size_t cap) {
    if (P % ORC_OCTETS_PAR_MACRO != 0 || N == 0 || N > 65535 || (geometrie != 1 && geometrie != 2)) return 0;
    const int ns = n_symboles(geometrie), spm = sous_pas(geometrie);
    uint32_t* cum = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)ntables * ns);
    for (int t = 0; t < ntables; ++t) {
        uint32_t c = 0;
        for (int s = 0; s < ns; ++s) {
            cum[t * ns + s] = c;
            c += freqs[t * ns + s];
        }
    }
    const size_t n_macro = P / ORC_OCTETS_PAR_MACRO;
    const size_t n_t = (n_macro + N - 1) / N;
    uint32_t* debuts = (uint32_t*)malloc(sizeof(uint32_t) * (n_t ? n_t : 1));
    uint32_t* etats = (uint32_t*)malloc(sizeof(uint32_t) * ORC_VOIES * (n_t ? n_t : 1));
    /* a symbol pushes at most one word: P*2 (g2) or P (g1) words bound the stream */
    const size_t max_mots = (size_t)P * (size_t)(spm / 4) + 1;
    uint16_t* mots = (uint16_t*)malloc(sizeof(uint16_t) * max_mots);
    uint16_t* pile = (uint16_t*)malloc(sizeof(uint16_t) * ((size_t)N * ORC_VOIES * spm + 1));
    size_t n_mots = 0;
    int erreur = 0;
    for (size_t t = 0; t < n_t && !erreur; ++t) {
        const size_t m0 = t * N;
        const size_t nb = (n_macro - m0) < N ? (n_macro - m0) : N;
        uint64_t x[ORC_VOIES];
        for (unsigned l = 0; l < ORC_VOIES; ++l) x[l] = ORC_L;
        size_t np = 0;
        for (size_t mm = nb; mm-- > 0;) {
            for (int k = spm; k-- > 0;) {
                for (int l = ORC_VOIES; l-- > 0;) {
                    const size_t n = ((m0 + mm) * ORC_VOIES + (size_t)l) * (size_t)spm + (size_t)k;
                    const int c = contexte(geometrie, kappa, n_kappa, n);
                    if (c >= ntables) {
                        erreur = 1;
                        break;
                    }
                    const int s = geometrie == 1 ? source[n] : (source[n / 2] >> (4 * (n % 2))) & 15;
                    const uint64_t f = freqs[c * ns + s];
                    if (f == 0) { /* rans.rs:319: symbol absent from its table */
                        erreur = 1;
                        break;
                    }
                    uint64_t xv = x[l];
                    if (xv >= (f << 20)) {
                        pile[np++] = (uint16_t)(xv & 0xFFFF);
                        xv >>= 16;
                    }
                    x[l] = ((xv / f) << 12) + (xv % f) + cum[c * ns + s];
                }
                if (erreur) break;
            }
            if (erreur) break;
        }
        debuts[t] = (uint32_t)n_mots;
        for (unsigned l = 0; l < ORC_VOIES; ++l) etats[t * ORC_VOIES + l] = (uint32_t)x[l];
        for (size_t i = 0; i < np; ++i) mots[n_mots + i] = pile[np - 1 - i]; /* reversed stack */
        n_mots += np;
    }
    size_t len = 0;
    if (!erreur) {
        len = ORC_ENTETE_FLUX + 4 * n_t + 4 * ORC_VOIES * n_t + 2 * n_mots;
        len = (len + 15) / 16 * 16;
        if (out && cap >= len) {
            memset(out, 0, len);
            wr32(out, (uint32_t)P);
            wr16(out + 4, N);
            out[6] = (uint8_t)geometrie;
            out[7] = 0;
            wr32(out + 8, (uint32_t)n_t);
            wr32(out + 12, (uint32_t)n_mots);
            uint8_t* p = out + ORC_ENTETE_FLUX;
            for (size_t t = 0; t < n_t; ++t, p += 4) wr32(p, debuts[t]);
            for (size_t i = 0; i < ORC_VOIES * n_t; ++i, p += 4) wr32(p, etats[i]);
            for (size_t i = 0; i < n_mots; ++i, p += 2) wr16(p, mots[i]);
        }
    }
    free(cum);
    free(debuts);
    free(etats);
    free(mots);
    free(pile);
    return len;
}

/* ---- decoder_avec, rans.rs:388-451 -------------------------------------------------------------- */
int orc_decoder(const orc_flux* f, const uint8_t* kappa, size_t n_kappa, const uint32_t* luts, int ntables,
                uint8_t* out, orc_bilan* bilan) {
    const int g = (int)f->geometrie, spm = sous_pas(g);
    const size_t p_octets = f->P;
    const size_t n_macro = p_octets / ORC_OCTETS_PAR_MACRO;
    memset(out, 0, p_octets);
    bilan->voies_hors_l = 0;
    bilan->tuiles_mots_faux = 0;
    bilan->premiere_tuile = -1;
    for (uint32_t t = 0; t < f->T; ++t) {
        const size_t m0 = (size_t)t * f->N;
        const size_t nb = (n_macro - m0) < f->N ? (n_macro - m0) : f->N;
        size_t p = rd32(f->debuts + 4 * t);
        const size_t fin = (t + 1 < f->T) ? rd32(f->debuts + 4 * (t + 1)) : f->W;
        int deborde = 0;
        uint32_t x[ORC_VOIES];
        for (unsigned l = 0; l < ORC_VOIES; ++l) x[l] = rd32(f->etats + 4 * ((size_t)t * ORC_VOIES + l));
        for (size_t m = 0; m < nb; ++m) {
            for (int k = 0; k < spm; ++k) {
                for (unsigned l = 0; l < ORC_VOIES; ++l) {
                    const size_t w = (m0 + m) * ORC_VOIES + l;
                    const size_t n = w * (size_t)spm + (size_t)k;
                    const int c = contexte(g, kappa, n_kappa, n);
                    if (c >= ntables) return -1; /* rans.rs:417: context without table */
                    const uint32_t xv = x[l];
                    const uint32_t e = luts[(size_t)c * ORC_M + (xv & (ORC_M - 1))];
                    uint32_t s, fr, b;
                    if (g == 1) {
                        s = e & 0xFF;
                        fr = ((e >> 8) & 0xFFF) + 1;
                        b = e >> 20;
                    } else {
                        s = e & 0xF;
                        fr = (e >> 4) & 0x1FFF;
                        b = e >> 17;
                    }
                    const uint32_t y = fr * (xv >> 12) + b; /* u32, wraps like the reference */
                    if (y < ORC_L) {
                        uint32_t mot = 0;
                        if (p < fin)
                            mot = rd16(f->mots + 2 * p);
                        else
                            deborde = 1;
                        x[l] = (y << 16) | mot;
                        ++p;
                    } else {
                        x[l] = y;
                    }
                    if (g == 1)
                        out[n] = (uint8_t)s;
                    else
                        out[n / 2] |= (uint8_t)(s << (4 * (n % 2)));
                }
            }
        }
        uint64_t hors = 0;
        for (unsigned l = 0; l < ORC_VOIES; ++l) hors += x[l] != ORC_L;
        const int mots_faux = deborde || p != fin;
        if (hors > 0 || mots_faux) {
            bilan->voies_hors_l += hors;
            bilan->tuiles_mots_faux += (uint64_t)mots_faux;
            if (bilan->premiere_tuile < 0) bilan->premiere_tuile = t;
        }
    }
    return 0;
}
