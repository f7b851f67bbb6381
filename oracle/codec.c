/*
 * codec.c — CPU restatement of the reference expert codec and part format (TEST INFRASTRUCTURE,
 * see oracle.h).
 *
 * Follows moteur/crates/trc-codec/src/lib.rs (matrix preparation, counts, v1.0/v1.2 coding,
 * reconstruction), moteur/crates/trc-format/src/lib.rs (part assembly / reading) and
 * moteur/crates/trc-noyaux/src/abi.rs (slot layout, LUTs of a layer).
 */
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

static inline uint32_t rd32(const uint8_t* p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24; }
static inline uint32_t rd16(const uint8_t* p) { return (uint32_t)p[0] | (uint32_t)p[1] << 8; }
static inline void wr32(uint8_t* p, uint32_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); p[2] = (uint8_t)(v >> 16); p[3] = (uint8_t)(v >> 24); }
static inline void wr16(uint8_t* p, uint32_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

#define SORTE_MEDIANES 0x01
#define SORTE_BIAIS 0x02
#define SORTE_DELTA 0x03
#define SORTE_CODES_CTX 0x04
#define CONTEXTE_AUCUN 0xFF

/* lib.rs:48-55 */
uint8_t orc_classe_echelle(uint8_t d) { return d < 128 ? 0 : (d == 128 ? 1 : 2); }

/* trc-format/src/lib.rs:67-77 */
uint8_t orc_canoniser_octet(uint8_t o) {
    uint8_t lo = o & 15, hi = o >> 4;
    if (lo == 8) lo = 0;
    if (hi == 8) hi = 0;
    return (uint8_t)(lo | (hi << 4));
}

static size_t pad128(size_t n) { return (n + 127) / 128 * 128; }

/* ---- preparer_matrice_avec, lib.rs:348-373 ---------------------------------------------------- */
void orc_preparer_matrice(const uint8_t* blocs, uint32_t R, uint32_t B, int canonique, uint8_t* medianes,
                          uint8_t* delta, uint8_t* qs) {
    const size_t nb = (size_t)R * B;
    memset(delta, 0, pad128(nb));
    memset(qs, 0, pad128(16 * nb));
    uint8_t* tri = (uint8_t*)malloc(B);
    for (uint32_t r = 0; r < R; ++r) {
        const uint8_t* ligne = blocs + (size_t)r * B * 17;
        for (uint32_t i = 0; i < B; ++i) tri[i] = ligne[17 * i];
        /* sort_unstable on u8 == counting order: any sort gives the same sequence */
        unsigned cnt[256] = {0};
        for (uint32_t i = 0; i < B; ++i) cnt[tri[i]]++;
        uint32_t k = 0;
        for (unsigned v = 0; v < 256; ++v)
            for (unsigned c = 0; c < cnt[v]; ++c) tri[k++] = (uint8_t)v;
        const uint8_t med = tri[B / 2];
        medianes[r] = med;
        for (uint32_t i = 0; i < B; ++i) {
            const size_t beta = (size_t)r * B + i;
            delta[beta] = (uint8_t)(ligne[17 * i] - med + 128);
            memcpy(qs + 16 * beta, ligne + 17 * i + 1, 16);
        }
    }
    free(tri);
    if (canonique)
        for (size_t i = 0; i < pad128(16 * nb); ++i) qs[i] = orc_canoniser_octet(qs[i]);
}

/* ---- ComptesMatrice::ajouter, lib.rs:390-398 -------------------------------------------------- */
void orc_comptes_ajouter(const uint8_t* delta, size_t n_delta, const uint8_t* qs, size_t n_qs, uint64_t* delta_c,
                         uint64_t* codes_c) {
    for (size_t i = 0; i < n_delta; ++i) delta_c[delta[i]]++;
    for (size_t n = 0; n < n_qs; ++n) {
        const size_t blk = n / 16;
        const uint8_t k = orc_classe_echelle(blk < n_delta ? delta[blk] : 0);
        codes_c[k * 256 + qs[n]]++;
    }
}

/* ---- ComptesMatrice over experts + tables(), lib.rs:378-413 ----------------------------------- */
void orc_tables_matrice(const uint8_t* const* blocs17, int n_experts, uint32_t R, uint32_t B, int canonique,
                        uint16_t* freqs_out) {
    const size_t nb = (size_t)R * B;
    uint64_t* dc = (uint64_t*)calloc(256, sizeof(uint64_t));
    uint64_t* cc = (uint64_t*)calloc(3 * 256, sizeof(uint64_t));
    uint8_t* med = (uint8_t*)malloc(R);
    uint8_t* delta = (uint8_t*)malloc(pad128(nb));
    uint8_t* qs = (uint8_t*)malloc(pad128(16 * nb));
    for (int x = 0; x < n_experts; ++x) {
        orc_preparer_matrice(blocs17[x], R, B, canonique, med, delta, qs);
        orc_comptes_ajouter(delta, pad128(nb), qs, pad128(16 * nb), dc, cc);
    }
    orc_table_depuis_comptes(dc, 1, freqs_out);
    for (int k = 0; k < 3; ++k) orc_table_depuis_comptes(cc + 256 * k, 1, freqs_out + 256 * (1 + k));
    free(dc);
    free(cc);
    free(med);
    free(delta);
    free(qs);
}

/* ---- assembler_partie, trc-format/src/lib.rs:879-910 ------------------------------------------ */
size_t orc_assembler_partie(uint16_t couche, uint16_t expert, uint8_t niveau, uint8_t n_matrices, int n_flux,
                            const uint8_t* sortes, const uint8_t* matrices, const uint8_t* contextes,
                            const uint32_t* produits, const uint8_t* const* octets, const uint32_t* longueurs,
                            uint8_t* out, size_t cap, uint32_t* utiles) {
    const size_t fin_table = 64 + 16 * (size_t)n_flux;
    size_t* dec = (size_t*)malloc(sizeof(size_t) * (n_flux ? n_flux : 1));
    size_t p = fin_table;
    for (int i = 0; i < n_flux; ++i) {
        p = (p + 15) / 16 * 16;
        dec[i] = p;
        p += longueurs[i];
    }
    const size_t u = p;
    const size_t total = (u + 4095) / 4096 * 4096;
    if (utiles) *utiles = (uint32_t)u;
    if (out && cap >= total) {
        memset(out, 0, total);
        static const uint32_t magie[2] = {0x30435254u, 0x31435254u};
        wr32(out, magie[niveau & 1]);
        wr16(out + 4, couche);
        wr16(out + 6, expert);
        out[8] = niveau;
        out[9] = n_matrices;
        wr16(out + 10, (uint32_t)n_flux);
        wr32(out + 12, (uint32_t)u);
        for (int i = 0; i < n_flux; ++i) {
            uint8_t* q = out + 64 + 16 * i;
            q[0] = sortes[i];
            q[1] = matrices[i];
            q[2] = contextes[i];
            wr32(q + 4, (uint32_t)dec[i]);
            wr32(q + 8, longueurs[i]);
            wr32(q + 12, produits[i]);
            memcpy(out + dec[i], octets[i], longueurs[i]);
        }
    }
    free(dec);
    return total;
}

/* ---- lire_partie, trc-format/src/lib.rs:813-877 ----------------------------------------------- */
static int sorte_connue(uint8_t s) {
    return s == 0x01 || s == 0x02 || s == 0x03 || s == 0x04 || s == 0x06 || s == 0x07 || s == 0x10 || s == 0x11 ||
           s == 0x12;
}

int orc_lire_partie(const uint8_t* o, size_t len, orc_partie* p) {
    if (len < 64) return -1;
    const uint32_t magie = rd32(o);
    const uint8_t niveau = o[8];
    if (niveau >= 2 || magie != (niveau == 0 ? 0x30435254u : 0x31435254u)) return -1;
    p->couche = (uint16_t)rd16(o + 4);
    p->expert = (uint16_t)rd16(o + 6);
    p->niveau = niveau;
    p->n_matrices = o[9];
    p->n_flux = rd16(o + 10);
    p->utiles = rd32(o + 12);
    for (int i = 16; i < 64; ++i)
        if (o[i]) return -1;
    if (p->utiles > len) return -1;
    const size_t fin_table = 64 + 16 * (size_t)p->n_flux;
    if (fin_table > p->utiles || p->n_flux > 64) return -1;
    uint64_t fin_prec = fin_table;
    for (uint32_t i = 0; i < p->n_flux; ++i) {
        const uint8_t* q = o + 64 + 16 * i;
        orc_desc_flux d;
        d.sorte = q[0];
        d.matrice = q[1];
        d.contexte = q[2];
        d.decalage = rd32(q + 4);
        d.longueur = rd32(q + 8);
        d.produits = rd32(q + 12);
        if (!sorte_connue(d.sorte)) return -1;
        if (q[3] != 0) return -1;
        if (d.matrice >= p->n_matrices) return -1;
        if (d.decalage % 16 != 0 || (uint64_t)d.decalage < fin_prec ||
            (uint64_t)d.decalage + d.longueur > (uint64_t)p->utiles)
            return -1;
        fin_prec = (uint64_t)d.decalage + d.longueur;
        p->flux[i] = d;
    }
    for (size_t i = p->utiles; i < len; ++i)
        if (o[i]) return -1;
    return 0;
}

static const orc_desc_flux* trouver(const orc_partie* p, uint8_t sorte, uint8_t j) {
    for (uint32_t i = 0; i < p->n_flux; ++i)
        if (p->flux[i].sorte == sorte && p->flux[i].matrice == j) return &p->flux[i];
    return NULL;
}

/* ---- coder_matrice_v10 for every matrix + assembler_partie, lib.rs:417-428 --------------------- */
size_t orc_coder_expert(uint16_t couche, uint16_t expert, int n_matrices, const uint32_t* R, const uint32_t* C,
                        const uint8_t* const* blocs17, const uint8_t* const* biais, const uint16_t* const* freqs,
                        int canonique, uint32_t N_delta, uint32_t N_codes, uint8_t* out, size_t cap,
                        uint32_t* utiles) {
    const int nf = 4 * n_matrices;
    uint8_t sortes[64] = {0}, mats[64] = {0}, ctxs[64] = {0};
    uint32_t prod[64] = {0}, lon[64] = {0};
    uint8_t* bufs[64] = {0};
    const uint8_t* octs[64] = {0};
    uint8_t* med_store[16] = {0};
    size_t total = 0;
    int ok = 1;
    for (int j = 0; j < n_matrices && ok; ++j) {
        const uint32_t B = C[j] / 32;
        const size_t nb = (size_t)R[j] * B;
        uint8_t* med = (uint8_t*)malloc(R[j]);
        uint8_t* delta = (uint8_t*)malloc(pad128(nb));
        uint8_t* qs = (uint8_t*)malloc(pad128(16 * nb));
        orc_preparer_matrice(blocs17[j], R[j], B, canonique, med, delta, qs);
        uint8_t* kappa = (uint8_t*)malloc(pad128(nb));
        for (size_t i = 0; i < pad128(nb); ++i) kappa[i] = orc_classe_echelle(delta[i]);
        const uint16_t* f = freqs[j];
        const size_t ld = orc_coder(delta, pad128(nb), 1, NULL, 0, f, 1, N_delta, NULL, 0);
        const size_t lc = orc_coder(qs, pad128(16 * nb), 1, kappa, pad128(nb), f + 256, 3, N_codes, NULL, 0);
        if (ld == 0 || lc == 0) ok = 0;
        uint8_t* fd = (uint8_t*)malloc(ld ? ld : 1);
        uint8_t* fc = (uint8_t*)malloc(lc ? lc : 1);
        if (ok) {
            orc_coder(delta, pad128(nb), 1, NULL, 0, f, 1, N_delta, fd, ld);
            orc_coder(qs, pad128(16 * nb), 1, kappa, pad128(nb), f + 256, 3, N_codes, fc, lc);
        }
        const int i0 = 4 * j;
        sortes[i0] = SORTE_MEDIANES; mats[i0] = (uint8_t)j; ctxs[i0] = CONTEXTE_AUCUN; prod[i0] = R[j]; lon[i0] = R[j];
        octs[i0] = med;
        sortes[i0 + 1] = SORTE_BIAIS; mats[i0 + 1] = (uint8_t)j; ctxs[i0 + 1] = CONTEXTE_AUCUN;
        prod[i0 + 1] = 4 * R[j]; lon[i0 + 1] = 4 * R[j]; octs[i0 + 1] = biais[j];
        sortes[i0 + 2] = SORTE_DELTA; mats[i0 + 2] = (uint8_t)j; ctxs[i0 + 2] = 0;
        prod[i0 + 2] = (uint32_t)pad128(nb); lon[i0 + 2] = (uint32_t)ld; octs[i0 + 2] = fd;
        sortes[i0 + 3] = SORTE_CODES_CTX; mats[i0 + 3] = (uint8_t)j; ctxs[i0 + 3] = CONTEXTE_AUCUN;
        prod[i0 + 3] = (uint32_t)pad128(16 * nb); lon[i0 + 3] = (uint32_t)lc; octs[i0 + 3] = fc;
        med_store[j] = med;
        bufs[i0 + 2] = fd;
        bufs[i0 + 3] = fc;
        free(delta);
        free(qs);
        free(kappa);
    }
    if (ok)
        total = orc_assembler_partie(couche, expert, 0, (uint8_t)n_matrices, nf, sortes, mats, ctxs, prod, octs, lon,
                                     out, cap, utiles);
    for (int j = 0; j < n_matrices; ++j) free(med_store[j]);
    for (int i = 0; i < nf; ++i) free(bufs[i]);
    return total;
}

/* ---- decoder_matrice_v10, lib.rs:190-218 ------------------------------------------------------- */
int orc_decoder_matrice(const uint8_t* partie, size_t len, uint8_t j, uint32_t R, uint32_t B,
                        const uint32_t* luts4, uint8_t* codes, uint8_t* echelles, uint8_t* biais,
                        orc_bilan* bd, orc_bilan* bc) {
    orc_partie p;
    if (orc_lire_partie(partie, len, &p) != 0) return -1;
    const size_t nb = (size_t)R * B;
    const orc_desc_flux* dm = trouver(&p, SORTE_MEDIANES, j);
    const orc_desc_flux* db = trouver(&p, SORTE_BIAIS, j);
    const orc_desc_flux* dd = trouver(&p, SORTE_DELTA, j);
    const orc_desc_flux* dc = trouver(&p, SORTE_CODES_CTX, j);
    if (!dm || !db || !dd || !dc) return -1;
    if (dm->longueur != R || dm->produits != R || db->longueur != 4 * R || db->produits != 4 * R) return -1;
    orc_flux fd, fc;
    if (orc_flux_lire(partie + dd->decalage, dd->longueur, &fd) != 0) return -1;
    if (orc_flux_lire(partie + dc->decalage, dc->longueur, &fc) != 0) return -1;
    if (fd.P != dd->produits || fc.P != dc->produits) return -1;
    if (fd.P != pad128(nb) || fc.P != pad128(16 * nb) || fd.geometrie != 1 || fc.geometrie != 1) return -1;
    uint8_t* delta = (uint8_t*)malloc(fd.P);
    uint8_t* tout = (uint8_t*)malloc(fc.P);
    orc_decoder(&fd, NULL, 0, luts4, 1, delta, bd);
    uint8_t* kappa = (uint8_t*)malloc(fd.P);
    for (size_t i = 0; i < fd.P; ++i) kappa[i] = orc_classe_echelle(delta[i]);
    const uint8_t* med = partie + dm->decalage;
    for (size_t beta = 0; beta < nb; ++beta) echelles[beta] = (uint8_t)(med[beta / B] + delta[beta] - 128);
    orc_decoder(&fc, kappa, fd.P, luts4 + ORC_M, 3, tout, bc);
    memcpy(codes, tout, 16 * nb);
    memcpy(biais, partie + db->decalage, 4 * R);
    free(delta);
    free(tout);
    free(kappa);
    return 0;
}

/* ---- slot layout, abi.rs:69-122 ---------------------------------------------------------------- */
static uint64_t al256(uint64_t x) { return (x + 255) & ~(uint64_t)255; }

orc_disposition orc_disposition_matrice(uint32_t lignes, uint32_t colonnes) {
    orc_disposition d;
    const uint64_t blocs = (uint64_t)lignes * (colonnes / 32);
    d.base = 0;
    d.echelles = al256(blocs * 16);
    d.biais = al256(d.echelles + blocs);
    d.pas = al256(d.biais + 4ull * lignes);
    return d;
}

uint64_t orc_taille_emplacement(const uint32_t* lignes, const uint32_t* colonnes) {
    uint64_t t = 0;
    for (int j = 0; j < 3; ++j) t += orc_disposition_matrice(lignes[j], colonnes[j]).pas;
    return t;
}

orc_disposition orc_disposition_j(const uint32_t* lignes, const uint32_t* colonnes, int j) {
    uint64_t base = 0;
    for (int i = 0; i < j; ++i) base += orc_disposition_matrice(lignes[i], colonnes[i]).pas;
    orc_disposition d = orc_disposition_matrice(lignes[j], colonnes[j]);
    d.base = base;
    return d;
}

/* ---- expert -> slot (decoder_partie lib.rs:223-260 into the SoA slot of abi.rs) --------------- */
int orc_decoder_expert(const uint8_t* partie, size_t len, const uint32_t* luts, const uint32_t* lignes,
                       const uint32_t* colonnes, uint8_t* emplacement, uint32_t* ctl) {
    ctl[0] = ctl[1] = ctl[2] = ctl[3] = 0;
    for (int j = 0; j < 3; ++j) {
        const uint32_t R = lignes[j], B = colonnes[j] / 32;
        const orc_disposition d = orc_disposition_j(lignes, colonnes, j);
        uint8_t* mat = emplacement + d.base;
        orc_bilan bd, bc;
        if (orc_decoder_matrice(partie, len, (uint8_t)j, R, B, luts + (size_t)j * 4 * ORC_M, mat, mat + d.echelles,
                                mat + d.biais, &bd, &bc) != 0) {
            ctl[1] += 1;
            continue;
        }
        ctl[0] += (uint32_t)(bd.voies_hors_l + bc.voies_hors_l);
        ctl[2] += (uint32_t)(bd.tuiles_mots_faux + bc.tuiles_mots_faux);
    }
    return 0;
}
