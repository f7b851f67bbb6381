// conteneur.cpp — the .trc v1.2 file container on the host: a reader that checks everything the
// reference reader checks before handing out tables and parts, and a writer for whole files.
//
// Format (decisions/ARCHITECTURE.md §4, trc-format/src/lib.rs): a fixed 4 096-byte header, then five
// sections aligned on 4 096 — MÉTA (GGUF v3 key/value pairs), RÉSIDENTS (table + data of the
// uncompressed tensors), TABLES (frequency tables per layer, matrix, stream kind, context),
// RÉPERTOIRE (64-byte entry per layer x expert) and TRONÇONS (the parts). Everything little-endian;
// every structure carries its size and its empreinte64. The reader refuses an unknown major
// version, stream kind or flag, non-zero reserved bytes, a wrong fingerprint and anything out of
// bounds, with the reference's refusal class (ErreurFormat, trc-format/src/lib.rs:129-148) as its
// status code.
//
// Reading uses pread on one descriptor (thread-safe: the streaming scheduler's readers share the
// open file); the writer buffers sequential writes and rewrites the reserved directory at the end.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "commun.hpp"
#include "empreinte.hpp"
#include "erreurs.hpp"

static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__, "the .trc format is little-endian");
static_assert(sizeof(trc_entree_repertoire) == 64, "directory entry: 64 bytes on disk");
static_assert(sizeof(trc_resident) == 128, "resident entry: 128 bytes on disk");
static_assert(sizeof(trc_desc_flux) == 16, "stream descriptor: 16 bytes on disk");

namespace {

constexpr uint8_t MAGIE[8] = {'T', 'R', 'O', 'N', 'C', 'O', 'N', 'S'};
constexpr uint64_t ALIGNEMENT = 4096;
constexpr uint64_t TAILLE_ENTETE = 4096;
constexpr uint16_t VERSION_MAJEURE = 1;
constexpr uint16_t VERSION_MINEURE = 2;
constexpr uint32_t DRAPEAUX_CONNUS =
    TRC_DRAPEAU_ALIGNE | TRC_DRAPEAU_NIVEAUX | TRC_DRAPEAU_BRUT | TRC_DRAPEAU_CANONIQUE | TRC_DRAPEAU_RAPIDE;
constexpr uint32_t MAGIE_PARTIE[2] = {0x30435254u, 0x31435254u};  // "TRC0", "TRC1"
constexpr uint64_t TAILLE_ENTETE_PARTIE = 64;
constexpr uint64_t TAILLE_DESC = 16;
constexpr uint64_t TAILLE_ENTREE = 64;
constexpr uint64_t TAILLE_RESIDENT = 128;
constexpr uint64_t ALIGNEMENT_RESIDENT = 256;

// A refusal: the status code of its class and the message.
struct Refus : std::runtime_error {
    int code;
    Refus(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] void refuser(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void refuser(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    throw Refus(code, buf);
}

// Runs f; turns a refusal into its status code and the thread's last-error message.
template <class F>
int garder(const char* quoi, F&& f) {
    try {
        f();
        return TRC_OK;
    } catch (const Refus& r) {
        ::trc::derniere_erreur() = std::string(quoi) + " : " + r.what();
        return r.code;
    } catch (const std::bad_alloc&) {
        ::trc::derniere_erreur() = std::string(quoi) + " : memoire epuisee";
        return TRC_FORMAT_ES;
    }
}

uint64_t aligner(uint64_t x, uint64_t a) { return (x + a - 1) / a * a; }

uint16_t lu16(const uint8_t* b) { uint16_t v; std::memcpy(&v, b, 2); return v; }
uint32_t lu32(const uint8_t* b) { uint32_t v; std::memcpy(&v, b, 4); return v; }
uint64_t lu64(const uint8_t* b) { uint64_t v; std::memcpy(&v, b, 8); return v; }
void eu16(uint8_t* b, uint16_t v) { std::memcpy(b, &v, 2); }
void eu32(uint8_t* b, uint32_t v) { std::memcpy(b, &v, 4); }
void eu64(uint8_t* b, uint64_t v) { std::memcpy(b, &v, 8); }

bool tout_nul(const uint8_t* b, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (b[i]) return false;
    return true;
}

// Stream kinds (trc-format/src/lib.rs:196-226): 0x05 is reserved ("not produced, not read").
bool sorte_connue(uint8_t s) {
    return s == 0x01 || s == 0x02 || s == 0x03 || s == 0x04 || s == 0x06 || s == 0x07 || s == 0x10 || s == 0x11 ||
           s == 0x12;
}

uint8_t lire_sorte(uint8_t s) {
    if (!sorte_connue(s)) refuser(TRC_FORMAT_SORTE, "sorte de flux inconnue : 0x%02x", s);
    return s;
}

// Bytes of a table payload by payload type (trc-format/src/lib.rs:535-542).
size_t octets_charge(uint8_t type) { return type == 1 ? 32 : type == 2 ? 512 : type == 3 ? 16 : 0; }

// ------------------------------------------------------------------------------ the header

// Entete::vers_octets (trc-format/src/lib.rs:289-322), fingerprint included.
void entete_vers_octets(const trc_entete_fichier& e, uint8_t* b) {
    std::memset(b, 0, TAILLE_ENTETE);
    std::memcpy(b, MAGIE, 8);
    eu16(b + 8, e.version_majeure);
    eu16(b + 10, e.version_mineure);
    eu32(b + 12, e.drapeaux);
    eu32(b + 16, uint32_t(ALIGNEMENT));
    eu32(b + 20, uint32_t(TAILLE_ENTETE));
    eu64(b + 24, e.taille_fichier);
    std::memcpy(b + 32, e.sha256_source, 32);
    eu64(b + 64, e.taille_source);
    eu16(b + 72, e.couches);
    eu16(b + 74, e.experts);
    eu16(b + 76, e.k);
    eu16(b + 78, e.matrices);
    for (int j = 0; j < 4; ++j) {
        eu32(b + 80 + 4 * j, e.lignes[j]);
        eu32(b + 96 + 4 * j, e.colonnes[j]);
    }
    eu32(b + 112, e.poids_par_bloc);
    eu32(b + 116, e.octets_par_bloc);
    b[120] = e.type_ggml;
    b[121] = e.niveaux;
    b[122] = e.classes_echelle;
    std::memcpy(b + 124, e.partition, 8);
    for (int i = 0; i < 8; ++i) {
        eu64(b + 136 + 16 * i, e.sections[i].decalage);
        eu64(b + 144 + 16 * i, e.sections[i].longueur);
    }
    eu64(b + 4088, trc::empreinte64(b, 4088));
}

// Entete::verifier_coherence (trc-format/src/lib.rs:392-439): levels against the NIVEAUX flag,
// CANONIQUE only from v1.2 on a one-level coded file, RAPIDE only from v1.2 on a one-level coded
// non-canonical file, 1 to 4 matrices, non-zero counts with k <= E, sections 5-7 all zero and
// sections 0-4 on a 4 096 boundary after the header.
void verifier_coherence(const trc_entete_fichier& e) {
    const bool brut = e.drapeaux & TRC_DRAPEAU_BRUT, canon = e.drapeaux & TRC_DRAPEAU_CANONIQUE,
               rapide = e.drapeaux & TRC_DRAPEAU_RAPIDE;
    if (e.niveaux < 1 || e.niveaux > 2) refuser(TRC_FORMAT_CHAMP, "nombre de niveaux : attendu 1 ou 2, lu %u", e.niveaux);
    if ((e.niveaux >= 2) != bool(e.drapeaux & TRC_DRAPEAU_NIVEAUX))
        refuser(TRC_FORMAT_DRAPEAUX, "drapeaux 0x%x : NIVEAUX contre %u niveaux", e.drapeaux, e.niveaux);
    if (e.version_mineure == 0 && e.niveaux != 1)
        refuser(TRC_FORMAT_CHAMP, "nombre de niveaux (v1.0) : attendu 1, lu %u", e.niveaux);
    if (brut && e.niveaux != 1) refuser(TRC_FORMAT_DRAPEAUX, "drapeaux 0x%x : BRUT a deux niveaux", e.drapeaux);
    if (canon && (e.version_mineure < 2 || brut || e.niveaux != 1))
        refuser(TRC_FORMAT_DRAPEAUX, "drapeaux 0x%x : CANONIQUE hors d'un fichier v1.2 code a un niveau", e.drapeaux);
    if (rapide && (e.version_mineure < 2 || brut || e.niveaux != 1 || canon))
        refuser(TRC_FORMAT_DRAPEAUX, "drapeaux 0x%x : RAPIDE hors d'un fichier v1.2 code, non canonique", e.drapeaux);
    if (e.matrices == 0 || e.matrices > 4)
        refuser(TRC_FORMAT_CHAMP, "matrices par expert : attendu 1 a 4, lu %u", e.matrices);
    for (unsigned j = e.matrices; j < 4; ++j)
        if (e.lignes[j] != 0 || e.colonnes[j] != 0) refuser(TRC_FORMAT_RESERVE, "dimensions de la matrice %u", j);
    if (e.couches == 0 || e.experts == 0 || e.k == 0 || e.k > e.experts)
        refuser(TRC_FORMAT_CHAMP, "couches, experts, k : attendu non nuls, k <= E, lu %u %u %u", e.couches, e.experts, e.k);
    for (int i = 0; i < 8; ++i) {
        const trc_section& s = e.sections[i];
        if (i >= 5) {
            if (s.decalage != 0 || s.longueur != 0) refuser(TRC_FORMAT_RESERVE, "section %d", i);
        } else if (s.decalage % ALIGNEMENT != 0 || s.decalage < TAILLE_ENTETE) {
            refuser(TRC_FORMAT_CHAMP, "decalage de la section %d : attendu multiple de 4096 apres l'en-tete, lu %llu", i,
                    (unsigned long long)s.decalage);
        }
    }
}

// Entete::depuis_octets (trc-format/src/lib.rs:325-390): magic, fingerprint, version, flags, fixed
// fields, reserved bytes, then coherence. The order decides which class a damaged header gets: a
// changed byte anywhere is first a fingerprint refusal.
trc_entete_fichier entete_depuis_octets(const uint8_t* b, size_t n) {
    if (n < TAILLE_ENTETE) refuser(TRC_FORMAT_LIMITES, "en-tete de %zu octets au lieu de 4096", n);
    if (std::memcmp(b, MAGIE, 8) != 0) refuser(TRC_FORMAT_MAGIE, "magie inconnue : ce n'est pas un fichier .trc");
    const uint64_t lue = lu64(b + 4088), calculee = trc::empreinte64(b, 4088);
    if (lue != calculee)
        refuser(TRC_FORMAT_EMPREINTE, "en-tete : lue 0x%016llx, calculee 0x%016llx", (unsigned long long)lue,
                (unsigned long long)calculee);
    trc_entete_fichier e;
    std::memset(&e, 0, sizeof(e));
    e.version_majeure = lu16(b + 8);
    e.version_mineure = lu16(b + 10);
    if (e.version_majeure != VERSION_MAJEURE || e.version_mineure > VERSION_MINEURE)
        refuser(TRC_FORMAT_VERSION, "version %u.%u non lue par ce lecteur (1.0 a 1.%u)", e.version_majeure,
                e.version_mineure, VERSION_MINEURE);
    e.drapeaux = lu32(b + 12);
    if ((e.drapeaux & ~DRAPEAUX_CONNUS) != 0 || (e.drapeaux & TRC_DRAPEAU_ALIGNE) == 0)
        refuser(TRC_FORMAT_DRAPEAUX, "drapeaux inconnus ou incoherents : 0x%x", e.drapeaux);
    if (lu32(b + 16) != ALIGNEMENT) refuser(TRC_FORMAT_CHAMP, "alignement : attendu 4096, lu %u", lu32(b + 16));
    if (lu32(b + 20) != TAILLE_ENTETE)
        refuser(TRC_FORMAT_CHAMP, "taille de l'en-tete : attendu 4096, lu %u", lu32(b + 20));
    if (b[123] != 0 || !tout_nul(b + 132, 4) || !tout_nul(b + 264, 4088 - 264))
        refuser(TRC_FORMAT_RESERVE, "octets reserves non nuls : en-tete");
    e.taille_fichier = lu64(b + 24);
    std::memcpy(e.sha256_source, b + 32, 32);
    e.taille_source = lu64(b + 64);
    e.couches = lu16(b + 72);
    e.experts = lu16(b + 74);
    e.k = lu16(b + 76);
    e.matrices = lu16(b + 78);
    for (int j = 0; j < 4; ++j) {
        e.lignes[j] = lu32(b + 80 + 4 * j);
        e.colonnes[j] = lu32(b + 96 + 4 * j);
    }
    e.poids_par_bloc = lu32(b + 112);
    e.octets_par_bloc = lu32(b + 116);
    e.type_ggml = b[120];
    e.niveaux = b[121];
    e.classes_echelle = b[122];
    std::memcpy(e.partition, b + 124, 8);
    for (int i = 0; i < 8; ++i) {
        e.sections[i].decalage = lu64(b + 136 + 16 * i);
        e.sections[i].longueur = lu64(b + 144 + 16 * i);
    }
    verifier_coherence(e);
    return e;
}

// ------------------------------------------------------------------- GGUF v3 key/value pairs

// A cursor over the pairs of the MÉTA section (GGUF v3 value types: 0 u8, 1 i8, 2 u16, 3 i16,
// 4 u32, 5 i32, 6 f32, 7 bool, 8 string, 9 array, 10 u64, 11 i64, 12 f64); restates the reading of
// trc-format/src/meta.rs:53-145. Arrays are skipped over, nested at most 4 deep.
struct Curseur {
    const uint8_t* b;
    uint64_t n, p;

    const uint8_t* prendre(uint64_t k) {
        if (k > n - p) refuser(TRC_FORMAT_LIMITES, "paire GGUF tronquee a l'octet %llu", (unsigned long long)p);
        const uint8_t* s = b + p;
        p += k;
        return s;
    }
    uint32_t u32() { return lu32(prendre(4)); }
    uint64_t u64() { return lu64(prendre(8)); }
    // A GGUF string: u64 length then the bytes, which must be UTF-8.
    uint64_t chaine(uint64_t& lg) {
        lg = u64();
        const uint8_t* s = prendre(lg);
        if (!utf8(s, lg)) refuser(TRC_FORMAT_LIMITES, "chaine GGUF non UTF-8 a l'octet %llu", (unsigned long long)p);
        return uint64_t(s - b);
    }
    static bool utf8(const uint8_t* s, uint64_t n) {
        for (uint64_t i = 0; i < n;) {
            const uint8_t c = s[i];
            uint32_t k, cp;
            if (c < 0x80) { ++i; continue; }
            if ((c & 0xE0) == 0xC0) { k = 1; cp = c & 0x1F; }
            else if ((c & 0xF0) == 0xE0) { k = 2; cp = c & 0x0F; }
            else if ((c & 0xF8) == 0xF0) { k = 3; cp = c & 0x07; }
            else return false;
            if (n - i <= k) return false;
            for (uint32_t t = 1; t <= k; ++t) {
                if ((s[i + t] & 0xC0) != 0x80) return false;
                cp = (cp << 6) | (s[i + t] & 0x3F);
            }
            // overlong forms, surrogates, beyond U+10FFFF
            if ((k == 1 && cp < 0x80) || (k == 2 && cp < 0x800) || (k == 3 && cp < 0x10000) || cp > 0x10FFFF ||
                (cp >= 0xD800 && cp <= 0xDFFF))
                return false;
            i += k + 1;
        }
        return true;
    }
    void scalaire(uint32_t t, trc_paire_meta& m) {
        switch (t) {
            case 0: m.u = prendre(1)[0]; break;
            case 1: m.i = int8_t(prendre(1)[0]); break;
            case 2: m.u = lu16(prendre(2)); break;
            case 3: m.i = int16_t(lu16(prendre(2))); break;
            case 4: m.u = u32(); break;
            case 5: m.i = int32_t(u32()); break;
            case 6: { float f; std::memcpy(&f, prendre(4), 4); m.f = f; break; }
            case 7: m.u = prendre(1)[0] != 0; break;
            case 8: m.chaine = chaine(m.n); break;
            case 10: m.u = u64(); break;
            case 11: m.i = int64_t(u64()); break;
            case 12: std::memcpy(&m.f, prendre(8), 8); break;
            default: refuser(TRC_FORMAT_CHAMP, "type de valeur GGUF : attendu 0 a 12, lu %u", t);
        }
    }
    // Skips one array value (after its type 9); returns its element type and count.
    void tableau(uint32_t profondeur, uint32_t& te, uint64_t& nb) {
        if (profondeur > 4) refuser(TRC_FORMAT_LIMITES, "tableaux GGUF imbriques trop profondement");
        te = u32();
        nb = u64();
        for (uint64_t i = 0; i < nb; ++i) {
            switch (te) {
                case 8: { uint64_t lg; chaine(lg); break; }
                case 9: { uint32_t t2; uint64_t n2; tableau(profondeur + 1, t2, n2); break; }
                case 0: case 1: case 7: prendre(1); break;
                case 2: case 3: prendre(2); break;
                case 4: case 5: case 6: prendre(4); break;
                case 10: case 11: case 12: prendre(8); break;
                default: refuser(TRC_FORMAT_CHAMP, "type d'element GGUF : attendu 0 a 12, lu %u", te);
            }
        }
    }
};

// lire_paires (trc-format/src/meta.rs:148-160): n pairs from the start of b; extents relative to b.
std::vector<trc_paire_meta> lire_paires(const uint8_t* b, uint64_t n_octets, uint64_t n) {
    Curseur c{b, n_octets, 0};
    std::vector<trc_paire_meta> v;
    for (uint64_t i = 0; i < n; ++i) {
        trc_paire_meta m;
        std::memset(&m, 0, sizeof(m));
        m.debut = c.p;
        m.cle = c.chaine(m.lg_cle);
        m.type = c.u32();
        if (m.type == 9) c.tableau(0, m.type_elem, m.n);
        else c.scalaire(m.type, m);
        m.fin = c.p;
        v.push_back(m);
    }
    return v;
}

// ------------------------------------------------------------------------------- the tables

// lire_tables (trc-format/src/lib.rs:586-658): count, reserved word, records [couche u16, matrice,
// sorte, contexte, payload type, u16 0, payload], fingerprint; layer and matrix within the header's
// counts; frequencies summing to 4 096, each <= 4 096; no bytes left over.
std::vector<trc_table> lire_tables(const uint8_t* b, uint64_t n_octets, const trc_entete_fichier& e) {
    if (n_octets < 16) refuser(TRC_FORMAT_LIMITES, "section TABLES trop courte");
    const uint64_t n_corps = n_octets - 8;
    if (trc::empreinte64(b, n_corps) != lu64(b + n_corps)) refuser(TRC_FORMAT_EMPREINTE, "section TABLES");
    const uint32_t n = lu32(b);
    if (lu32(b + 4) != 0) refuser(TRC_FORMAT_RESERVE, "en-tete de TABLES");
    uint64_t p = 8;
    std::vector<trc_table> v;
    for (uint32_t i = 0; i < n; ++i) {
        if (p + 8 > n_corps) refuser(TRC_FORMAT_LIMITES, "enregistrement de table %u", i);
        trc_table t;
        std::memset(&t, 0, sizeof(t));
        t.couche = lu16(b + p);
        t.matrice = b[p + 2];
        t.sorte = lire_sorte(b[p + 3]);
        t.contexte = b[p + 4];
        t.type_charge = b[p + 5];
        if (lu16(b + p + 6) != 0) refuser(TRC_FORMAT_RESERVE, "enregistrement de table %u", i);
        const size_t taille = octets_charge(t.type_charge);
        if (taille == 0) refuser(TRC_FORMAT_CHAMP, "type de charge : attendu 1, 2 ou 3, lu %u", t.type_charge);
        p += 8;
        if (p + taille > n_corps) refuser(TRC_FORMAT_LIMITES, "charge de la table %u", i);
        if (t.couche >= e.couches || t.matrice >= e.matrices)
            refuser(TRC_FORMAT_CHAMP, "table : (couche, matrice) attendu < (%u, %u), lu (%u, %u)", e.couches, e.matrices,
                    t.couche, t.matrice);
        std::memcpy(&t.charge, b + p, taille);
        if (t.type_charge != 3) {
            const unsigned nf = t.type_charge == 1 ? 16 : 256;
            uint32_t somme = 0;
            bool trop = false;
            for (unsigned s = 0; s < nf; ++s) {
                somme += t.charge.frequences[s];
                trop |= t.charge.frequences[s] > 4096;
            }
            if (somme != 4096 || trop)
                refuser(TRC_FORMAT_CHAMP, "somme des frequences de la table %u : attendu 4096, lu %u", i, somme);
        }
        p += taille;
        v.push_back(t);
    }
    if (p != n_corps) refuser(TRC_FORMAT_LIMITES, "octets en trop dans la section TABLES");
    return v;
}

// verifier_tables_canoniques (trc-format/src/lib.rs:661-680): on a CANONIQUE file every CODES_CTX
// table has 256 frequencies and gives 0 to the 31 bytes that carry a nibble 8 (-0 never coded).
void verifier_tables_canoniques(const std::vector<trc_table>& tables) {
    for (const trc_table& t : tables) {
        if (t.sorte != TRC_SORTE_CODES_CTX) continue;
        if (t.type_charge != 2)
            refuser(TRC_FORMAT_CHAMP, "charge d'une table CODES_CTX : attendu 256 frequences (type 2), lu %u",
                    t.type_charge);
        for (unsigned s = 0; s < 256; ++s)
            if (((s & 0xF) == 8 || (s >> 4) == 8) && t.charge.frequences[s] != 0)
                refuser(TRC_FORMAT_CHAMP,
                        "table CODES_CTX (%u, %u, contexte %u) d'un fichier canonique : octet 0x%02x de frequence %u",
                        t.couche, t.matrice, t.contexte, s, t.charge.frequences[s]);
    }
}

bool table_avant(const trc_table& a, const trc_table& b) {
    if (a.couche != b.couche) return a.couche < b.couche;
    if (a.matrice != b.matrice) return a.matrice < b.matrice;
    if (a.sorte != b.sorte) return a.sorte < b.sorte;
    return a.contexte < b.contexte;
}

// --------------------------------------------------------------------------- resident tensors

// lire_table_residents (trc-format/src/lib.rs:738-777): count, reserved word, 128-byte entries with
// a NUL-padded UTF-8 name, offsets on 256, 1 to 4 dimensions.
std::vector<trc_resident> lire_table_residents(const uint8_t* b, uint64_t n_octets) {
    const uint32_t n = lu32(b);
    if (lu32(b + 4) != 0) refuser(TRC_FORMAT_RESERVE, "en-tete de RESIDENTS");
    if (n_octets < 8 + TAILLE_RESIDENT * n) refuser(TRC_FORMAT_LIMITES, "table des residents");
    std::vector<trc_resident> v(n);
    for (uint32_t i = 0; i < n; ++i) {
        trc_resident& r = v[i];
        std::memcpy(&r, b + 8 + TAILLE_RESIDENT * i, TAILLE_RESIDENT);
        const size_t lg = strnlen(r.nom, 64);
        if (!tout_nul(reinterpret_cast<const uint8_t*>(r.nom) + lg, 64 - lg))
            refuser(TRC_FORMAT_RESERVE, "nom du resident %u", i);
        if (!Curseur::utf8(reinterpret_cast<const uint8_t*>(r.nom), lg))
            refuser(TRC_FORMAT_CHAMP, "nom de resident %u : attendu UTF-8", i);
        if (r.decalage % ALIGNEMENT_RESIDENT != 0 || r.n_dims == 0 || r.n_dims > 4)
            refuser(TRC_FORMAT_CHAMP, "resident %.64s : decalage multiple de 256, 1 a 4 dimensions, lu %llu %u", r.nom,
                    (unsigned long long)r.decalage, r.n_dims);
    }
    return v;
}

uint64_t debut_zone_residents(uint64_t n) { return aligner(8 + TAILLE_RESIDENT * n, ALIGNEMENT); }

// ----------------------------------------------------------------------------------- a part

// lire_partie (trc-format/src/lib.rs:813-866): 64-byte header (magic by level, layer, expert, level,
// n_matrices, n_streams, useful bytes, 48 zero bytes), 16-byte descriptors (kind, matrix, fixed
// context, 0, offset, length, produced) with offsets on 16, in order, inside the useful bytes, and
// zero padding after them.
void lire_partie(const uint8_t* o, uint64_t n, trc_partie_info& info) {
    if (n < TAILLE_ENTETE_PARTIE) refuser(TRC_FORMAT_LIMITES, "partie de troncon plus courte que son en-tete");
    const uint32_t magie = lu32(o);
    const uint8_t niveau = o[8];
    if (niveau >= 2 || magie != MAGIE_PARTIE[niveau])
        refuser(TRC_FORMAT_CHAMP, "magie de partie : attendu TRC0 ou TRC1 selon le niveau, lu 0x%08x, niveau %u", magie,
                niveau);
    std::memset(&info, 0, sizeof(info));
    info.couche = lu16(o + 4);
    info.expert = lu16(o + 6);
    info.niveau = niveau;
    info.n_matrices = o[9];
    info.n_flux = lu16(o + 10);
    info.utiles = lu32(o + 12);
    if (!tout_nul(o + 16, 48)) refuser(TRC_FORMAT_RESERVE, "en-tete de partie");
    if (info.utiles > n)
        refuser(TRC_FORMAT_LIMITES, "partie : %u octets utiles annonces, %llu presents", info.utiles,
                (unsigned long long)n);
    const uint64_t fin_table = TAILLE_ENTETE_PARTIE + TAILLE_DESC * info.n_flux;
    if (fin_table > info.utiles) refuser(TRC_FORMAT_LIMITES, "table des flux hors de la partie");
    uint64_t fin_prec = fin_table;
    for (uint32_t i = 0; i < info.n_flux; ++i) {
        trc_desc_flux d;
        std::memcpy(&d, o + TAILLE_ENTETE_PARTIE + TAILLE_DESC * i, TAILLE_DESC);
        lire_sorte(d.sorte);
        if (d.reserve != 0) refuser(TRC_FORMAT_RESERVE, "descripteur du flux %u", i);
        if (d.matrice >= info.n_matrices)
            refuser(TRC_FORMAT_CHAMP, "matrice du flux %u : attendu < %u, lu %u", i, info.n_matrices, d.matrice);
        if (d.decalage % 16 != 0 || d.decalage < fin_prec || uint64_t(d.decalage) + d.longueur > info.utiles)
            refuser(TRC_FORMAT_LIMITES, "flux %u : decalage %u, longueur %u", i, d.decalage, d.longueur);
        fin_prec = uint64_t(d.decalage) + d.longueur;
    }
    if (!tout_nul(o + info.utiles, n - info.utiles)) refuser(TRC_FORMAT_RESERVE, "bourrage de la partie");
}

// ------------------------------------------------------------------------------- file access

struct Descripteur {
    int fd = -1;
    ~Descripteur() {
        if (fd >= 0) ::close(fd);
    }
};

void lire_a(int fd, uint64_t decalage, uint64_t n, void* dst) {
    uint8_t* d = static_cast<uint8_t*>(dst);
    while (n > 0) {
        const size_t k = size_t(std::min<uint64_t>(n, uint64_t(1) << 30));
        const ssize_t r = ::pread(fd, d, k, off_t(decalage));
        if (r < 0) refuser(TRC_FORMAT_ES, "lecture a %llu : %s", (unsigned long long)decalage, std::strerror(errno));
        if (r == 0) refuser(TRC_FORMAT_ES, "lecture a %llu : fin de fichier", (unsigned long long)decalage);
        d += r;
        decalage += uint64_t(r);
        n -= uint64_t(r);
    }
}

}  // namespace

// ====================================================================================== reader

struct trc_fichier {
    Descripteur f;
    std::string chemin;
    trc_entete_fichier entete;
    std::vector<uint8_t> meta;  // u64 n, then the pairs (fingerprint excluded)
    std::vector<trc_paire_meta> paires;
    std::vector<trc_resident> residents;
    uint64_t debut_donnees = 0;
    std::vector<trc_table> tables;  // sorted by (couche, matrice, sorte, contexte)
    std::vector<std::pair<uint32_t, uint32_t>> index_tables;
    std::vector<trc_entree_repertoire> repertoire;
    uint64_t octets_lus = 0;

    std::vector<uint8_t> lire(uint64_t decalage, uint64_t n) {
        std::vector<uint8_t> v(n);
        lire_a(f.fd, decalage, n, v.data());
        octets_lus += n;
        return v;
    }
};

namespace {

// Fichier::ouvrir (trc-format/src/lib.rs:957-1090): header, file size, sections in bounds and not
// overlapping, MÉTA, resident table, TABLES, RÉPERTOIRE; neither resident data nor parts are read.
void ouvrir(trc_fichier& F, const char* chemin) {
    F.chemin = chemin;
    F.f.fd = ::open(chemin, O_RDONLY | O_CLOEXEC);
    if (F.f.fd < 0) refuser(TRC_FORMAT_ES, "ouverture de %s : %s", chemin, std::strerror(errno));
    struct stat st;
    if (::fstat(F.f.fd, &st) != 0) refuser(TRC_FORMAT_ES, "fstat : %s", std::strerror(errno));
    const uint64_t taille = uint64_t(st.st_size);
    const std::vector<uint8_t> tete = F.lire(0, TAILLE_ENTETE);
    F.entete = entete_depuis_octets(tete.data(), tete.size());
    const trc_entete_fichier& e = F.entete;
    if (e.taille_fichier != taille)
        refuser(TRC_FORMAT_CHAMP, "taille du fichier : attendu %llu, lu %llu", (unsigned long long)e.taille_fichier,
                (unsigned long long)taille);
    trc_section s[5];
    for (int i = 0; i < 5; ++i) {
        s[i] = e.sections[i];
        if (s[i].longueur > taille || s[i].decalage > taille - s[i].longueur)
            refuser(TRC_FORMAT_LIMITES, "section %d au-dela de la fin du fichier", i);
    }
    std::sort(s, s + 5, [](const trc_section& a, const trc_section& b) { return a.decalage < b.decalage; });
    for (int i = 0; i + 1 < 5; ++i)
        if (s[i].decalage + s[i].longueur > s[i + 1].decalage) refuser(TRC_FORMAT_LIMITES, "sections qui se chevauchent");

    // MÉTA: u64 n, the pairs, the fingerprint of both
    const trc_section sm = e.sections[TRC_SECTION_META];
    std::vector<uint8_t> mb = F.lire(sm.decalage, sm.longueur);
    if (mb.size() < 16) refuser(TRC_FORMAT_LIMITES, "section META");
    const uint64_t n_paires = lu64(mb.data());
    F.paires = lire_paires(mb.data() + 8, mb.size() - 16, n_paires);
    const uint64_t fin_paires = 8 + (F.paires.empty() ? 0 : F.paires.back().fin);
    if (fin_paires != mb.size() - 8) refuser(TRC_FORMAT_LIMITES, "octets en trop dans la section META");
    if (trc::empreinte64(mb.data(), fin_paires) != lu64(mb.data() + fin_paires))
        refuser(TRC_FORMAT_EMPREINTE, "section META");
    mb.resize(fin_paires);
    F.meta = std::move(mb);

    // RÉSIDENTS: the table, zeros up to 4 096, the data zone, the table's fingerprint in the last 8 bytes
    const trc_section sr = e.sections[TRC_SECTION_RESIDENTS];
    if (sr.longueur < 16) refuser(TRC_FORMAT_LIMITES, "section RESIDENTS");
    const uint32_t n_res = lu32(F.lire(sr.decalage, 8).data());
    const uint64_t lg_table = 8 + TAILLE_RESIDENT * uint64_t(n_res);
    const uint64_t debut_zone = debut_zone_residents(n_res);
    if (debut_zone + 8 > sr.longueur) refuser(TRC_FORMAT_LIMITES, "table des residents plus longue que sa section");
    const std::vector<uint8_t> table_r = F.lire(sr.decalage, lg_table);
    const uint64_t e_table = lu64(F.lire(sr.decalage + sr.longueur - 8, 8).data());
    if (trc::empreinte64(table_r.data(), table_r.size()) != e_table)
        refuser(TRC_FORMAT_EMPREINTE, "table des residents");
    const std::vector<uint8_t> bourrage = F.lire(sr.decalage + lg_table, debut_zone - lg_table);
    if (!tout_nul(bourrage.data(), bourrage.size()))
        refuser(TRC_FORMAT_RESERVE, "bourrage de la table des residents");
    F.residents = lire_table_residents(table_r.data(), table_r.size());
    uint64_t fin_zone = 0;
    for (const trc_resident& r : F.residents) fin_zone = std::max(fin_zone, r.decalage + r.octets);
    if (debut_zone + fin_zone + 8 != sr.longueur)
        refuser(TRC_FORMAT_CHAMP, "longueur de RESIDENTS : attendu %llu, lu %llu",
                (unsigned long long)(debut_zone + fin_zone + 8), (unsigned long long)sr.longueur);
    F.debut_donnees = sr.decalage + debut_zone;

    // TABLES, sorted; one per (couche, matrice, sorte, contexte); canonical check on CANONIQUE files
    const trc_section stb = e.sections[TRC_SECTION_TABLES];
    const std::vector<uint8_t> tb = F.lire(stb.decalage, stb.longueur);
    F.tables = lire_tables(tb.data(), tb.size(), e);
    std::stable_sort(F.tables.begin(), F.tables.end(), table_avant);
    const uint32_t nm = e.matrices;
    F.index_tables.assign(size_t(e.couches) * nm, {0u, 0u});
    for (uint32_t i = 0; i < F.tables.size();) {
        uint32_t j = i;
        while (j < F.tables.size() && F.tables[j].couche == F.tables[i].couche &&
               F.tables[j].matrice == F.tables[i].matrice)
            ++j;
        F.index_tables[size_t(F.tables[i].couche) * nm + F.tables[i].matrice] = {i, j};
        i = j;
    }
    for (size_t i = 0; i + 1 < F.tables.size(); ++i) {
        const trc_table &a = F.tables[i], &b = F.tables[i + 1];
        if (!table_avant(a, b))
            refuser(TRC_FORMAT_CHAMP, "tables : une seule par (couche, matrice, sorte, contexte), lu (%u, %u, 0x%02x, %u) deux fois",
                    a.couche, a.matrice, a.sorte, a.contexte);
    }
    if (e.drapeaux & TRC_DRAPEAU_CANONIQUE) verifier_tables_canoniques(F.tables);

    // RÉPERTOIRE: couches x experts entries in (couche, expert) order, then their fingerprint
    const trc_section sd = e.sections[TRC_SECTION_REPERTOIRE];
    const uint64_t n_ent = uint64_t(e.couches) * e.experts;
    if (sd.longueur != n_ent * TAILLE_ENTREE + 8)
        refuser(TRC_FORMAT_CHAMP, "longueur du REPERTOIRE : attendu %llu, lu %llu",
                (unsigned long long)(n_ent * TAILLE_ENTREE + 8), (unsigned long long)sd.longueur);
    const std::vector<uint8_t> rb = F.lire(sd.decalage, sd.longueur);
    const uint64_t n_corps = n_ent * TAILLE_ENTREE;
    if (trc::empreinte64(rb.data(), n_corps) != lu64(rb.data() + n_corps))
        refuser(TRC_FORMAT_EMPREINTE, "section REPERTOIRE");
    const trc_section stc = e.sections[TRC_SECTION_TRONCONS];
    const bool canon = e.drapeaux & TRC_DRAPEAU_CANONIQUE;
    F.repertoire.resize(n_ent);
    for (uint64_t i = 0; i < n_ent; ++i) {
        trc_entree_repertoire& en = F.repertoire[i];
        std::memcpy(&en, rb.data() + i * TAILLE_ENTREE, TAILLE_ENTREE);
        if (en.reserve != 0) refuser(TRC_FORMAT_RESERVE, "entree %llu du repertoire", (unsigned long long)i);
        const uint16_t c = uint16_t(i / e.experts), x = uint16_t(i % e.experts);
        if (en.couche != c || en.expert != x)
            refuser(TRC_FORMAT_CHAMP, "entree %llu du repertoire : attendu (%u, %u), lu (%u, %u)", (unsigned long long)i, c,
                    x, en.couche, en.expert);
        const uint64_t total = uint64_t(en.longueur[0]) + en.longueur[1];
        const bool ok = en.decalage % ALIGNEMENT == 0 && en.longueur[0] % ALIGNEMENT == 0 &&
                        en.longueur[1] % ALIGNEMENT == 0 && en.utiles[0] <= en.longueur[0] &&
                        en.utiles[1] <= en.longueur[1] && en.longueur[0] > 0 && en.decalage >= stc.decalage &&
                        en.decalage + total <= stc.decalage + stc.longueur &&
                        (e.niveaux >= 2 || (en.longueur[1] == 0 && en.utiles[1] == 0 && en.empreinte_niveau[1] == 0)) &&
                        (canon || en.empreinte_canonique == 0);
        if (!ok)
            refuser(TRC_FORMAT_LIMITES, "entree (%u, %u) du repertoire : decalage %llu, longueurs %u %u, utiles %u %u", c, x,
                    (unsigned long long)en.decalage, en.longueur[0], en.longueur[1], en.utiles[0], en.utiles[1]);
    }
}

const trc_table* chercher_table(const trc_fichier& F, uint16_t couche, uint8_t matrice, uint8_t sorte, uint8_t ctx) {
    if (couche >= F.entete.couches || matrice >= F.entete.matrices) return nullptr;
    const auto r = F.index_tables[size_t(couche) * F.entete.matrices + matrice];
    for (uint32_t i = r.first; i < r.second; ++i)
        if (F.tables[i].sorte == sorte && F.tables[i].contexte == ctx) return &F.tables[i];
    return nullptr;
}

// verifier_partie (trc-codec/src/lib.rs:264-275) plus the structure and identity checks of
// reconstruire_avec (:286-297): the useful bytes hash to the directory's level fingerprint, the part
// reads, and it is the part of (couche, expert, niveau) with the directory's useful-byte count.
void verifier_partie(const trc_fichier& F, uint16_t couche, uint16_t expert, uint32_t niveau, const uint8_t* o,
                     uint64_t n) {
    const trc_entree_repertoire& en = F.repertoire[size_t(couche) * F.entete.experts + expert];
    const uint32_t u = en.utiles[niveau];
    if (n < u)
        refuser(TRC_FORMAT_LIMITES, "partie de niveau %u de (%u, %u) : %llu octets, %u utiles attendus", niveau, couche,
                expert, (unsigned long long)n, u);
    const uint64_t h = trc::empreinte64(o, u);
    if (h != en.empreinte_niveau[niveau])
        refuser(TRC_FORMAT_EMPREINTE, "partie de niveau %u de (%u, %u) : 0x%016llx au lieu de 0x%016llx", niveau, couche,
                expert, (unsigned long long)h, (unsigned long long)en.empreinte_niveau[niveau]);
    trc_partie_info info;
    lire_partie(o, std::min<uint64_t>(n, aligner(u, ALIGNEMENT)), info);
    if (info.couche != couche || info.expert != expert || info.niveau != niveau)
        refuser(TRC_FORMAT_CHAMP, "la partie porte (%u, %u, niveau %u) au lieu de (%u, %u, niveau %u)", info.couche,
                info.expert, info.niveau, couche, expert, niveau);
    if (info.utiles != u)
        refuser(TRC_FORMAT_CHAMP, "octets utiles de la partie %u, repertoire %u", info.utiles, u);
}

}  // namespace

// ====================================================================================== writer

struct trc_ecrivain {
    Descripteur f;
    std::vector<uint8_t> tampon;
    uint64_t position = 0;    // bytes written so far (buffered included)
    uint64_t ecrit_fd = 0;    // bytes already handed to the descriptor
    trc_section sections[8] = {};
    // 0 created, 1 MÉTA written, 2 RÉSIDENTS written, 3 TABLES written (before TRONÇONS),
    // 4 TRONÇONS open, 5 TABLES written after TRONÇONS (which it closed)
    int etape = 0;
    bool tables_ecrites = false;
    uint16_t couches = 0, experts = 0;
    uint64_t debut_repertoire = 0;
    std::vector<trc_entree_repertoire> repertoire;
    std::vector<uint8_t> present;

    void vider() {
        uint64_t fait = 0;
        while (fait < tampon.size()) {
            const ssize_t r = ::pwrite(f.fd, tampon.data() + fait, tampon.size() - fait, off_t(ecrit_fd + fait));
            if (r < 0) refuser(TRC_FORMAT_ES, "ecriture : %s", std::strerror(errno));
            fait += uint64_t(r);
        }
        ecrit_fd += tampon.size();
        tampon.clear();
    }
    void ecrire(const void* p, uint64_t n) {
        const uint8_t* o = static_cast<const uint8_t*>(p);
        position += n;
        while (n > 0) {
            const uint64_t k = std::min<uint64_t>(n, (uint64_t(8) << 20) - tampon.size());
            tampon.insert(tampon.end(), o, o + k);
            o += k;
            n -= k;
            if (tampon.size() >= (uint64_t(8) << 20)) vider();
        }
    }
    void zeros(uint64_t n) {
        static const uint8_t z[4096] = {0};
        while (n > 0) {
            const uint64_t k = std::min<uint64_t>(n, sizeof(z));
            ecrire(z, k);
            n -= k;
        }
    }
    void aligner_sur(uint64_t a) { zeros(aligner(position, a) - position); }
    uint64_t ouvrir_section() {
        aligner_sur(ALIGNEMENT);
        return position;
    }
    void reecrire(uint64_t decalage, const void* p, uint64_t n) {
        vider();
        const uint8_t* o = static_cast<const uint8_t*>(p);
        while (n > 0) {
            const ssize_t r = ::pwrite(f.fd, o, n, off_t(decalage));
            if (r < 0) refuser(TRC_FORMAT_ES, "reecriture : %s", std::strerror(errno));
            o += r;
            decalage += uint64_t(r);
            n -= uint64_t(r);
        }
    }
};

namespace {

void etape(trc_ecrivain* w, int attendue, const char* quoi, int ou = -1) {
    if (w == nullptr) refuser(TRC_ERREUR_USAGE, "ecrivain nul");
    if (w->etape != attendue && w->etape != ou)
        refuser(TRC_ERREUR_USAGE, "%s hors d'ordre (MÉTA, RÉSIDENTS, TABLES avant ou apres TRONÇONS, terminer)", quoi);
}

}  // namespace

// ====================================================================================== C-ABI

extern "C" {

uint64_t trc_empreinte64(const void* octets, uint64_t n) {
    return trc::empreinte64(static_cast<const uint8_t*>(octets), size_t(n));
}

void trc_sha256(const void* octets, uint64_t n, uint8_t sortie[32]) {
    trc::Sha256 s;
    s.ajouter(static_cast<const uint8_t*>(octets), size_t(n));
    s.finir(sortie);
}

// empreinte64 of an expert (ARCHITECTURE.md §4.11-4.12): for j = 0, 1, 2 its 17-byte blocks
// [e, qs16] in beta order, then for j = 0, 1, 2 its f32 biases.
uint64_t trc_empreinte_expert(const uint8_t* const* blocs17, const float* const* biais, const trc_dims_expert* dims) {
    trc::Sha256 s;
    for (int j = 0; j < 3; ++j)
        s.ajouter(blocs17[j], size_t(dims->lignes[j]) * (dims->colonnes[j] / 32) * 17);
    for (int j = 0; j < 3; ++j) s.ajouter(reinterpret_cast<const uint8_t*>(biais[j]), size_t(dims->lignes[j]) * 4);
    uint8_t d[32];
    s.finir(d);
    return trc::empreinte64_de(d);
}

// empreinte_emplacement (trc-ordo/src/lib.rs:238-262): the same fingerprint recomputed from a
// decoded SoA slot (scales, codes and biases at the slot disposition of each matrix).
uint64_t trc_empreinte_emplacement(const uint8_t* emplacement, const trc_dims_expert* dims) {
    trc::Sha256 s;
    std::vector<uint8_t> v;
    for (uint32_t j = 0; j < 3; ++j) {
        const trc_disposition d = trc::disposition(*dims, j);
        const uint64_t n = uint64_t(dims->lignes[j]) * (dims->colonnes[j] / 32);
        v.resize(17 * n);
        for (uint64_t beta = 0; beta < n; ++beta) {
            v[17 * beta] = emplacement[d.base + d.echelles + beta];
            std::memcpy(&v[17 * beta + 1], emplacement + d.base + 16 * beta, 16);
        }
        s.ajouter(v.data(), v.size());
    }
    for (uint32_t j = 0; j < 3; ++j) {
        const trc_disposition d = trc::disposition(*dims, j);
        s.ajouter(emplacement + d.base + d.biais, size_t(dims->lignes[j]) * 4);
    }
    uint8_t dd[32];
    s.finir(dd);
    return trc::empreinte64_de(dd);
}

int trc_partie_lire(const uint8_t* octets, uint64_t n, trc_partie_info* info) {
    if (octets == nullptr || info == nullptr) return trc::usage("pointeur nul");
    return garder("partie", [&] { lire_partie(octets, n, *info); });
}

// ------------------------------------------------------------------------------------ reader

int trc_fichier_ouvrir(const char* chemin, trc_fichier** sortie) {
    if (chemin == nullptr || sortie == nullptr) return trc::usage("pointeur nul");
    *sortie = nullptr;
    auto F = std::make_unique<trc_fichier>();
    const int r = garder(chemin, [&] { ouvrir(*F, chemin); });
    if (r == TRC_OK) *sortie = F.release();
    return r;
}

void trc_fichier_fermer(trc_fichier* f) { delete f; }

const trc_entete_fichier* trc_fichier_entete(const trc_fichier* f) { return &f->entete; }

uint64_t trc_fichier_meta(const trc_fichier* f, const uint8_t** octets) {
    if (octets) *octets = f->meta.data();
    return f->meta.size();
}

uint64_t trc_fichier_n_paires(const trc_fichier* f) { return f->paires.size(); }

const trc_paire_meta* trc_fichier_paires(const trc_fichier* f) { return f->paires.data(); }

int64_t trc_fichier_chercher_paire(const trc_fichier* f, const char* cle) {
    const size_t n = std::strlen(cle);
    const uint8_t* base = f->meta.data() + 8;
    for (size_t i = 0; i < f->paires.size(); ++i) {
        const trc_paire_meta& p = f->paires[i];
        if (p.lg_cle == n && std::memcmp(base + p.cle, cle, n) == 0) return int64_t(i);
    }
    return -1;
}

uint32_t trc_fichier_n_residents(const trc_fichier* f) { return uint32_t(f->residents.size()); }

const trc_resident* trc_fichier_residents(const trc_fichier* f) { return f->residents.data(); }

uint64_t trc_fichier_debut_donnees(const trc_fichier* f) { return f->debut_donnees; }

uint32_t trc_fichier_n_tables(const trc_fichier* f) { return uint32_t(f->tables.size()); }

const trc_table* trc_fichier_tables(const trc_fichier* f) { return f->tables.data(); }

const trc_table* trc_fichier_table(const trc_fichier* f, uint16_t couche, uint8_t matrice, uint8_t sorte,
                                   uint8_t contexte) {
    return chercher_table(*f, couche, matrice, sorte, contexte);
}

// luts_couche (trc-ordo/src/lib.rs:265-273): the frequencies a layer's LUTs are built from, for
// j = 0..2: DELTA context 0, CODES_CTX contexts 0, 1, 2 (u16[3][4][256], ready for trc_luts_couche).
int trc_fichier_freqs_couche(const trc_fichier* f, uint16_t couche, uint16_t* freqs) {
    if (f == nullptr || freqs == nullptr) return trc::usage("pointeur nul");
    if (couche >= f->entete.couches) return trc::usage("couche %u hors du fichier (%u)", couche, f->entete.couches);
    if (f->entete.matrices != 3) return trc::usage("%u matrices par expert, 3 attendues", f->entete.matrices);
    const uint8_t sortes[4] = {TRC_SORTE_DELTA, TRC_SORTE_CODES_CTX, TRC_SORTE_CODES_CTX, TRC_SORTE_CODES_CTX};
    const uint8_t ctx[4] = {0, 0, 1, 2};
    for (uint8_t j = 0; j < 3; ++j)
        for (int t = 0; t < 4; ++t) {
            const trc_table* tb = chercher_table(*f, couche, j, sortes[t], ctx[t]);
            if (tb == nullptr || tb->type_charge != 2)
                return trc::usage("table (%u, %u, 0x%02x, %u) absente ou pas de 256 frequences", couche, j, sortes[t], ctx[t]);
            std::memcpy(freqs + (size_t(j) * 4 + t) * 256, tb->charge.frequences, 512);
        }
    return TRC_OK;
}

const trc_entree_repertoire* trc_fichier_repertoire(const trc_fichier* f) { return f->repertoire.data(); }

const trc_entree_repertoire* trc_fichier_entree(const trc_fichier* f, uint16_t couche, uint16_t expert) {
    if (couche >= f->entete.couches || expert >= f->entete.experts) return nullptr;
    return &f->repertoire[size_t(couche) * f->entete.experts + expert];
}

uint64_t trc_fichier_octets_lus(const trc_fichier* f) { return f->octets_lus; }

int trc_fichier_lire(const trc_fichier* f, uint64_t decalage, uint64_t octets, void* dst) {
    if (f == nullptr || (dst == nullptr && octets)) return trc::usage("pointeur nul");
    if (decalage > f->entete.taille_fichier || octets > f->entete.taille_fichier - decalage)
        return trc::usage("lecture [%llu, +%llu) hors du fichier", (unsigned long long)decalage,
                          (unsigned long long)octets);
    return garder("lecture", [&] { lire_a(f->f.fd, decalage, octets, dst); });
}

// Reads levels 0 .. niveaux-1 of (couche, expert) in one request (EntreeRepertoire::longueur_jusqua,
// trc-format/src/lib.rs:497-500) into dst; with verifier, checks each level as verifier_partie does.
int trc_fichier_lire_partie(const trc_fichier* f, uint16_t couche, uint16_t expert, uint32_t niveaux, void* dst,
                            uint64_t cap, int verifier, uint64_t* octets) {
    if (f == nullptr || dst == nullptr) return trc::usage("pointeur nul");
    if (couche >= f->entete.couches || expert >= f->entete.experts)
        return trc::usage("(%u, %u) hors du fichier", couche, expert);
    if (niveaux == 0 || niveaux > f->entete.niveaux) return trc::usage("%u niveaux demandes, %u dans le fichier", niveaux, f->entete.niveaux);
    const trc_entree_repertoire& en = f->repertoire[size_t(couche) * f->entete.experts + expert];
    uint64_t n = 0;
    for (uint32_t l = 0; l < niveaux; ++l) n += en.longueur[l];
    if (cap < n) return trc::usage("tampon de %llu octets, %llu a lire", (unsigned long long)cap, (unsigned long long)n);
    if (octets) *octets = n;
    return garder("partie", [&] {
        lire_a(f->f.fd, en.decalage, n, dst);
        if (verifier) {
            const uint8_t* o = static_cast<const uint8_t*>(dst);
            for (uint32_t l = 0; l < niveaux; ++l) {
                verifier_partie(*f, couche, expert, l, o, en.longueur[l]);
                o += en.longueur[l];
            }
        }
    });
}

int trc_fichier_verifier_partie(const trc_fichier* f, uint16_t couche, uint16_t expert, uint32_t niveau,
                                const uint8_t* octets, uint64_t n) {
    if (f == nullptr || octets == nullptr) return trc::usage("pointeur nul");
    if (couche >= f->entete.couches || expert >= f->entete.experts || niveau >= f->entete.niveaux)
        return trc::usage("(%u, %u, niveau %u) hors du fichier", couche, expert, niveau);
    return garder("partie", [&] { verifier_partie(*f, couche, expert, niveau, octets, n); });
}

// ------------------------------------------------------------------------------------ writer

trc_ecrivain* trc_ecrivain_creer(const char* chemin) {
    if (chemin == nullptr) {
        trc::usage("chemin nul");
        return nullptr;
    }
    auto w = std::make_unique<trc_ecrivain>();
    w->f.fd = ::open(chemin, O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644);
    if (w->f.fd < 0) {
        trc::derniere_erreur() = std::string("creation de ") + chemin + " : " + std::strerror(errno);
        return nullptr;
    }
    w->tampon.reserve(size_t(8) << 20);
    w->zeros(TAILLE_ENTETE);  // the header, written last
    return w.release();
}

void trc_ecrivain_abandonner(trc_ecrivain* w) { delete w; }

// serialiser_meta (trc-format/src/lib.rs:915-926): u64 n, the pairs, the fingerprint. The pairs
// (any already-serialised GGUF v3 pairs, additions included) must read back as exactly n pairs.
int trc_ecrivain_meta(trc_ecrivain* w, const uint8_t* paires, uint64_t octets, uint64_t n_paires) {
    return garder("MÉTA", [&] {
        etape(w, 0, "MÉTA");
        if (paires == nullptr && octets) refuser(TRC_ERREUR_USAGE, "paires nulles");
        uint64_t fin = 0;
        try {
            const auto v = lire_paires(paires, octets, n_paires);
            fin = v.empty() ? 0 : v.back().fin;
        } catch (const Refus& r) {
            refuser(TRC_ERREUR_USAGE, "paires GGUF illisibles : %s", r.what());
        }
        if (fin != octets)
            refuser(TRC_ERREUR_USAGE, "%llu paires ne couvrent pas %llu octets", (unsigned long long)n_paires,
                    (unsigned long long)octets);
        std::vector<uint8_t> b(8 + octets + 8);
        eu64(b.data(), n_paires);
        if (octets) std::memcpy(b.data() + 8, paires, octets);
        eu64(b.data() + 8 + octets, trc::empreinte64(b.data(), 8 + octets));
        const uint64_t d = w->ouvrir_section();
        w->ecrire(b.data(), b.size());
        w->sections[TRC_SECTION_META] = {d, w->position - d};
        w->etape = 1;
    });
}

// RÉSIDENTS (disposer_residents, serialiser_table_residents, trc-format/src/lib.rs:696-735): the
// tensors laid out in the given order on 256-byte boundaries of the data zone; decalage and
// empreinte of each entry are filled in here.
int trc_ecrivain_residents(trc_ecrivain* w, trc_resident* residents, const uint8_t* const* donnees, uint32_t n) {
    return garder("RÉSIDENTS", [&] {
        etape(w, 1, "RÉSIDENTS");
        if (n && (residents == nullptr || donnees == nullptr)) refuser(TRC_ERREUR_USAGE, "residents nuls");
        uint64_t p = 0;
        for (uint32_t i = 0; i < n; ++i) {
            trc_resident& r = residents[i];
            const size_t lg = strnlen(r.nom, 64);
            if (!tout_nul(reinterpret_cast<const uint8_t*>(r.nom) + lg, 64 - lg) ||
                !Curseur::utf8(reinterpret_cast<const uint8_t*>(r.nom), lg))
                refuser(TRC_ERREUR_USAGE, "nom du resident %u : au plus 64 octets UTF-8 sans zero", i);
            if (r.n_dims == 0 || r.n_dims > 4) refuser(TRC_ERREUR_USAGE, "resident %u : %u dimensions", i, r.n_dims);
            p = aligner(p, ALIGNEMENT_RESIDENT);
            r.decalage = p;
            r.empreinte = trc::empreinte64(donnees[i], r.octets);
            p += r.octets;
        }
        std::vector<uint8_t> table(8 + TAILLE_RESIDENT * n, 0);
        eu32(table.data(), n);
        if (n) std::memcpy(table.data() + 8, residents, TAILLE_RESIDENT * n);
        const uint64_t d = w->ouvrir_section();
        w->ecrire(table.data(), table.size());
        w->aligner_sur(ALIGNEMENT);
        const uint64_t zone = w->position;
        for (uint32_t i = 0; i < n; ++i) {
            w->zeros(zone + residents[i].decalage - w->position);
            w->ecrire(donnees[i], residents[i].octets);
        }
        const uint64_t e = trc::empreinte64(table.data(), table.size());
        w->ecrire(&e, 8);
        w->sections[TRC_SECTION_RESIDENTS] = {d, w->position - d};
        w->etape = 2;
    });
}

// serialiser_tables (trc-format/src/lib.rs:563-583): count, reserved word, records in the given
// order, fingerprint. Kinds and payload types are checked; frequencies are left to the reader.
// Called before trc_ecrivain_troncons, or after the last part (it then closes TRONÇONS and the
// TABLES section follows it: an encoder that learns its tables layer by layer writes them last).
int trc_ecrivain_tables(trc_ecrivain* w, const trc_table* tables, uint32_t n) {
    return garder("TABLES", [&] {
        etape(w, 2, "TABLES", 4);
        if (n && tables == nullptr) refuser(TRC_ERREUR_USAGE, "tables nulles");
        std::vector<uint8_t> b(8, 0);
        eu32(b.data(), n);
        for (uint32_t i = 0; i < n; ++i) {
            const trc_table& t = tables[i];
            if (!sorte_connue(t.sorte)) refuser(TRC_ERREUR_USAGE, "table %u : sorte 0x%02x", i, t.sorte);
            const size_t taille = octets_charge(t.type_charge);
            if (taille == 0) refuser(TRC_ERREUR_USAGE, "table %u : type de charge %u", i, t.type_charge);
            uint8_t r[8];
            eu16(r, t.couche);
            r[2] = t.matrice;
            r[3] = t.sorte;
            r[4] = t.contexte;
            r[5] = t.type_charge;
            eu16(r + 6, 0);
            b.insert(b.end(), r, r + 8);
            const uint8_t* c = reinterpret_cast<const uint8_t*>(&t.charge);
            b.insert(b.end(), c, c + taille);
        }
        const uint64_t e = trc::empreinte64(b.data(), b.size());
        b.resize(b.size() + 8);
        eu64(b.data() + b.size() - 8, e);
        if (w->etape == 4) {
            trc_section& st = w->sections[TRC_SECTION_TRONCONS];
            st.longueur = w->position - st.decalage;
        }
        const uint64_t d = w->ouvrir_section();
        w->ecrire(b.data(), b.size());
        w->sections[TRC_SECTION_TABLES] = {d, w->position - d};
        w->tables_ecrites = true;
        w->etape = w->etape == 4 ? 5 : 3;
    });
}

// Reserves the RÉPERTOIRE (couches x experts entries + fingerprint) and opens TRONÇONS.
int trc_ecrivain_troncons(trc_ecrivain* w, uint16_t couches, uint16_t experts) {
    return garder("TRONÇONS", [&] {
        etape(w, 2, "TRONÇONS", 3);
        if (couches == 0 || experts == 0) refuser(TRC_ERREUR_USAGE, "couches et experts non nuls");
        const uint64_t n = uint64_t(couches) * experts;
        w->couches = couches;
        w->experts = experts;
        w->debut_repertoire = w->ouvrir_section();
        w->zeros(n * TAILLE_ENTREE + 8);
        w->sections[TRC_SECTION_REPERTOIRE] = {w->debut_repertoire, n * TAILLE_ENTREE + 8};
        const uint64_t d = w->ouvrir_section();
        w->sections[TRC_SECTION_TRONCONS] = {d, 0};
        w->repertoire.assign(n, trc_entree_repertoire{});
        w->present.assign(n, 0);
        w->etape = 4;
    });
}

// One expert's parts: level 0 (and level 1 right after it on two-level files), each checked with
// lire_partie, written up to its useful bytes and padded with zeros to 4 096. The directory entry
// (offset, lengths, useful bytes, level fingerprints, plus the caller's origin and canonical
// fingerprints) is returned in `ecrite` when not NULL.
int trc_ecrivain_partie(trc_ecrivain* w, uint16_t couche, uint16_t expert, const uint8_t* niveau0, uint64_t octets0,
                        const uint8_t* niveau1, uint64_t octets1, uint64_t empreinte_origine,
                        uint64_t empreinte_canonique, trc_entree_repertoire* ecrite) {
    return garder("partie", [&] {
        etape(w, 4, "partie");
        if (couche >= w->couches || expert >= w->experts)
            refuser(TRC_ERREUR_USAGE, "(%u, %u) hors de %u x %u", couche, expert, w->couches, w->experts);
        const size_t i = size_t(couche) * w->experts + expert;
        if (w->present[i]) refuser(TRC_ERREUR_USAGE, "partie (%u, %u) deja ecrite", couche, expert);
        if (niveau0 == nullptr) refuser(TRC_ERREUR_USAGE, "niveau 0 nul");
        trc_entree_repertoire en{};
        en.decalage = w->position;
        en.couche = couche;
        en.expert = expert;
        en.empreinte_origine = empreinte_origine;
        en.empreinte_canonique = empreinte_canonique;
        const uint8_t* niv[2] = {niveau0, niveau1};
        const uint64_t oct[2] = {octets0, octets1};
        for (uint32_t l = 0; l < 2 && niv[l] != nullptr; ++l) {
            trc_partie_info info;
            lire_partie(niv[l], oct[l], info);
            if (info.couche != couche || info.expert != expert || info.niveau != l)
                refuser(TRC_ERREUR_USAGE, "la partie porte (%u, %u, niveau %u) au lieu de (%u, %u, niveau %u)", info.couche,
                        info.expert, info.niveau, couche, expert, l);
            en.utiles[l] = info.utiles;
            en.longueur[l] = uint32_t(aligner(info.utiles, ALIGNEMENT));
            en.empreinte_niveau[l] = trc::empreinte64(niv[l], info.utiles);
            w->ecrire(niv[l], info.utiles);
            w->aligner_sur(ALIGNEMENT);
        }
        w->repertoire[i] = en;
        w->present[i] = 1;
        if (ecrite) *ecrite = en;
    });
}

// Closes TRONÇONS, writes the directory and its fingerprint into the reserved zone, then the
// header (sections, file size, fingerprint), after verifier_coherence (Ecrivain::terminer,
// trc-format/src/lib.rs:1227-1239). The writer is freed whatever the outcome.
int trc_ecrivain_terminer(trc_ecrivain* w, const trc_entete_fichier* entete, uint64_t* taille) {
    std::unique_ptr<trc_ecrivain> garde(w);
    return garder("terminer", [&] {
        etape(w, 4, "terminer", 5);
        if (!w->tables_ecrites) refuser(TRC_ERREUR_USAGE, "TABLES jamais ecrites");
        if (entete == nullptr) refuser(TRC_ERREUR_USAGE, "en-tete nul");
        for (size_t i = 0; i < w->present.size(); ++i)
            if (!w->present[i])
                refuser(TRC_ERREUR_USAGE, "partie (%zu, %zu) jamais ecrite", i / w->experts, i % w->experts);
        if (entete->couches != w->couches || entete->experts != w->experts)
            refuser(TRC_ERREUR_USAGE, "en-tete %u x %u, troncons %u x %u", entete->couches, entete->experts, w->couches,
                    w->experts);
        if (w->etape == 4) {
            trc_section& st = w->sections[TRC_SECTION_TRONCONS];
            st.longueur = w->position - st.decalage;
        }
        w->aligner_sur(ALIGNEMENT);
        const uint64_t n = w->repertoire.size() * TAILLE_ENTREE;
        std::vector<uint8_t> rb(n + 8);
        std::memcpy(rb.data(), w->repertoire.data(), n);
        eu64(rb.data() + n, trc::empreinte64(rb.data(), n));
        trc_entete_fichier e = *entete;
        std::memcpy(e.sections, w->sections, sizeof(e.sections));
        e.taille_fichier = w->position;
        verifier_coherence(e);
        w->reecrire(w->debut_repertoire, rb.data(), rb.size());
        std::vector<uint8_t> tete(TAILLE_ENTETE);
        entete_vers_octets(e, tete.data());
        w->reecrire(0, tete.data(), tete.size());
        if (::fsync(w->f.fd) != 0) refuser(TRC_FORMAT_ES, "fsync : %s", std::strerror(errno));
        if (taille) *taille = e.taille_fichier;
    });
}

}  // extern "C"
