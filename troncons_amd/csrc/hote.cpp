// hote.cpp — host-side helpers of the C-ABI (no device needed): slot layout, decoder grids and the
// geometry-1 LUTs of a layer, restated from moteur/crates/trc-noyaux/src/abi.rs.
#include <cstring>
#include <string>

#include "commun.hpp"
#include "erreurs.hpp"

namespace trc {
std::string& derniere_erreur() {
    thread_local std::string message;
    return message;
}
int& dernier_code_hip() {
    thread_local int code = 0;
    return code;
}
}  // namespace trc

using trc::usage;

extern "C" const char* trc_derniere_erreur(void) { return trc::derniere_erreur().c_str(); }

extern "C" int trc_dernier_code_hip(void) { return trc::dernier_code_hip(); }

extern "C" trc_disposition trc_disposition_matrice(uint32_t lignes, uint32_t colonnes) {
    return trc::disposition_matrice(lignes, colonnes);
}

extern "C" int trc_dims_verifier(const trc_dims_expert* dims) {
    if (dims == nullptr) return usage("dims absent");
    for (int j = 0; j < 3; ++j) {
        const uint32_t r = dims->lignes[j], c = dims->colonnes[j];
        if (r == 0 || c == 0 || c % 32 != 0)
            return usage("matrice %d : forme %u x %u (colonnes multiples de 32 exigees)", j, r, c);
        if (uint64_t(r) * (c / 32) * 16 > 0xFFFFFFFFull) return usage("matrice %d : plus de 4 Gio de codes", j);
    }
    return TRC_OK;
}

extern "C" trc_disposition trc_disposition_j(const trc_dims_expert* dims, uint32_t j) {
    return trc::disposition(*dims, j);
}

extern "C" uint64_t trc_taille_emplacement(const trc_dims_expert* dims) {
    uint64_t t = 0;
    for (int j = 0; j < 3; ++j) t += trc::disposition_matrice(dims->lignes[j], dims->colonnes[j]).pas;
    return t;
}

static uint32_t tuiles(uint64_t octets) {
    const uint64_t macro = (octets + 127) / 128;
    return uint32_t((macro + trc::MACRO_PAR_TUILE - 1) / trc::MACRO_PAR_TUILE);
}

static uint32_t au_moins_1(uint32_t v) { return v > 0 ? v : 1; }

// abi.rs:137-141: one DELTA tile per 32-lane half-block unit of FILS_ECHELLES/32 tiles, one
// CODES_CTX tile per FILS_CODES/32.
extern "C" void trc_grilles_decodeur(const trc_dims_expert* dims, uint32_t g1[3], uint32_t g2[3]) {
    uint32_t td = 0, tc = 0;
    for (int j = 0; j < 3; ++j) {
        const uint64_t blocs = uint64_t(dims->lignes[j]) * (dims->colonnes[j] / 32);
        td = td > tuiles(blocs) ? td : tuiles(blocs);
        tc = tc > tuiles(16 * blocs) ? tc : tuiles(16 * blocs);
    }
    const uint32_t pe = trc::FILS_ECHELLES / 32, pc = trc::FILS_CODES / 32;
    g1[0] = au_moins_1((td + pe - 1) / pe);
    g1[1] = 3;
    g1[2] = 1;
    g2[0] = au_moins_1((tc + pc - 1) / pc);
    g2[1] = 3;
    g2[2] = 1;
}

// abi.rs:149-176: T of every DELTA and CODES_CTX stream read from a host copy of the part.
extern "C" int trc_grilles_depuis_partie(const uint8_t* partie, size_t octets, uint32_t g1[3], uint32_t g2[3]) {
    auto lu16 = [&](size_t p, uint32_t& v) -> bool {
        if (p + 2 > octets) return false;
        v = uint32_t(partie[p]) | uint32_t(partie[p + 1]) << 8;
        return true;
    };
    auto lu32 = [&](size_t p, uint32_t& v) -> bool {
        if (p + 4 > octets) return false;
        v = uint32_t(partie[p]) | uint32_t(partie[p + 1]) << 8 | uint32_t(partie[p + 2]) << 16 |
            uint32_t(partie[p + 3]) << 24;
        return true;
    };
    if (partie == nullptr) return usage("partie absente");
    uint32_t n_flux;
    if (!lu16(10, n_flux)) return usage("partie de moins de 12 o");
    uint32_t td = 0, tc = 0;
    bool vus[3][2] = {{false, false}, {false, false}, {false, false}};
    for (uint32_t i = 0; i < n_flux; ++i) {
        const size_t e = 64 + 16 * size_t(i);
        if (e + 2 > octets) return usage("table des flux tronquee");
        const uint8_t sorte = partie[e];
        const uint32_t j = partie[e + 1];
        int k;
        if (sorte == 0x03)
            k = 0;
        else if (sorte == 0x04)
            k = 1;
        else
            continue;
        if (j > 2) return usage("flux %u : matrice %u", i, j);
        uint32_t dec, t;
        if (!lu32(e + 4, dec)) return usage("table des flux tronquee");
        if (!lu32(size_t(dec) + 8, t)) return usage("flux %u hors de la partie", i);
        vus[j][k] = true;
        if (k == 0)
            td = td > t ? td : t;
        else
            tc = tc > t ? tc : t;
    }
    for (int j = 0; j < 3; ++j)
        if (!vus[j][0] || !vus[j][1]) return usage("DELTA ou CODES_CTX absent pour une matrice");
    const uint32_t pe = trc::FILS_ECHELLES / 32, pc = trc::FILS_CODES / 32;
    g1[0] = au_moins_1((td + pe - 1) / pe);
    g1[1] = 3;
    g1[2] = 1;
    g2[0] = au_moins_1((tc + pc - 1) / pc);
    g2[1] = 3;
    g2[2] = 1;
    return TRC_OK;
}

// abi.rs:179-182: at most 96 blocks per matrix
extern "C" void trc_grille_brut(const trc_dims_expert* dims, uint32_t g[3]) {
    uint64_t n = 1;
    for (int j = 0; j < 3; ++j) {
        const uint64_t b = uint64_t(dims->lignes[j]) * (dims->colonnes[j] / 32);
        n = n > b ? n : b;
    }
    uint64_t x = (n + trc::FILS_BRUT - 1) / trc::FILS_BRUT;
    g[0] = uint32_t(x < 1 ? 1 : (x > 96 ? 96 : x));
    g[1] = 3;
    g[2] = 1;
}

// abi.rs:187-204: lut[i] = s | (f-1) << 8 | (i - c[s]) << 20 for i in [c[s], c[s] + f[s]).
extern "C" int trc_lut_geometrie1(const uint16_t* freq, size_t n, uint32_t* lut) {
    if (freq == nullptr || lut == nullptr) return usage("pointeur nul");
    if (n != 256) return usage("%zu frequences, 256 attendues", n);
    uint32_t somme = 0;
    for (int s = 0; s < 256; ++s) somme += freq[s];
    if (somme != 4096) return usage("somme des frequences %u, 4 096 attendus", somme);
    uint32_t c = 0;
    for (uint32_t s = 0; s < 256; ++s) {
        const uint32_t f = freq[s];
        for (uint32_t i = c; i < c + f; ++i) lut[i] = s | ((f - 1) << 8) | ((i - c) << 20);
        c += f;
    }
    return TRC_OK;
}

// abi.rs:210-221: [j][0] DELTA, [j][1 + kappa] CODES_CTX; an absent table is a zero LUT.
extern "C" int trc_luts_couche(const uint16_t* const* freqs, uint32_t* luts) {
    if (freqs == nullptr || luts == nullptr) return usage("pointeur nul");
    std::memset(luts, 0, sizeof(uint32_t) * trc::LUTS_PAR_COUCHE);
    for (int j = 0; j < 3; ++j)
        for (int t = 0; t < 4; ++t)
            if (freqs[j * 4 + t] != nullptr) {
                const int r = trc_lut_geometrie1(freqs[j * 4 + t], 256, luts + size_t(j * 4 + t) * 4096);
                if (r != TRC_OK) return usage("matrice %d, table %d : %s", j, t, trc::derniere_erreur().c_str() + 8);
            }
    return TRC_OK;
}
