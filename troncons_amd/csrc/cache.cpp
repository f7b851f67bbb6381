// cache.cpp — the expert slot cache of the streaming path and its simulator (host C++).
//
// Role of moteur/crates/trc-cache (decisions/ARCHITECTURE.md §5.7). Two stages:
//   - VRAM: `emplacements` slots of DECODED experts (the SoA slot, 13 254 144 bytes for gpt-oss);
//   - warm RAM: `tiedes` entries of CODED parts in pinned host memory (0: none).
// A VRAM miss served by RAM costs a copy and a decode, not a read. The simulator (trc_cache_rejouer)
// is this same code driven by a routing trace, so an engine's counters can be compared with it to
// the unit.
//
// A VRAM slot: Libre --(miss)--> EnVol --(pret: decode done)--> Present --(eviction)--> Libre.
// An EnVol slot is never evicted (the decoder writes into it); the experts a layer in progress
// asked for are pinned until trc_cache_liberer_couche and are never evicted either. Behaviour rules
// (trc-cache/src/lib.rs:23-47): all experts of a request are pinned before the first is served;
// the RAM stage is inclusive and sees every access (a VRAM hit also touches the RAM entry); a RAM
// entry is only created by a disk read; `evictions` counts VRAM evictions.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <functional>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "erreurs.hpp"

namespace {

using Id = uint32_t;  // (couche << 16) | expert
inline Id id_de(uint16_t c, uint16_t e) { return (uint32_t(c) << 16) | e; }
constexpr uint32_t NUL = 0xFFFFFFFFu;
constexpr uint64_t JAMAIS = ~uint64_t(0);

// ----------------------------------------------------------------------------- the trace

// A routing trace: choix[(t * L + l) * k + i] is the i-th expert chosen by layer l at token t
// (trc-cache/src/trace.rs:24-45).
struct Trace {
    uint16_t experts = 0, couches = 0, k = 0;
    uint32_t jetons = 0;
    std::vector<uint16_t> choix;
    const uint16_t* groupe(uint32_t t, uint32_t l) const { return &choix[(size_t(t) * couches + l) * k]; }
};

// --------------------------------------------------------------------------- the policies

// Replacement policy contract (trc-cache/src/politiques.rs:13-24): it holds an order over the
// present ids only; the cache reports each hit (acceder), entry (inserer) and exit (retirer);
// victime names the id to evict among the non-pinned ones without removing it.
struct Politique {
    virtual ~Politique() = default;
    virtual void acceder(Id id, uint64_t t) = 0;
    virtual void inserer(Id id, uint64_t t) = 0;
    virtual void retirer(Id id) = 0;
    virtual bool victime(const std::function<bool(Id)>& epingle, Id& v) = 0;
};

// LRU: evict the least recently used non-pinned id. A doubly linked list in arrays plus an
// id -> node map: O(1) accesses; victime walks from the oldest and skips pinned ids (at most the
// experts of the layers in progress). The order depends only on the order of calls: the k experts
// of one layer share their t and rank in service order. With `fifo`, hits do not refresh (FIFO).
struct Lru final : Politique {
    struct Noeud {
        Id id;
        uint32_t prec, suiv;
    };
    std::vector<Noeud> noeuds;
    std::vector<uint32_t> libres;
    std::unordered_map<Id, uint32_t> index;
    uint32_t tete = NUL, queue = NUL;  // oldest, newest
    bool fifo;
    explicit Lru(bool f = false) : fifo(f) {}

    void detacher(uint32_t i) {
        const Noeud n = noeuds[i];
        (n.prec == NUL ? tete : noeuds[n.prec].suiv) = n.suiv;
        (n.suiv == NUL ? queue : noeuds[n.suiv].prec) = n.prec;
    }
    void accrocher(uint32_t i) {
        noeuds[i].prec = queue;
        noeuds[i].suiv = NUL;
        (queue == NUL ? tete : noeuds[queue].suiv) = i;
        queue = i;
    }
    void acceder(Id id, uint64_t) override {
        if (fifo) return;
        const uint32_t i = index.at(id);
        if (i != queue) {
            detacher(i);
            accrocher(i);
        }
    }
    void inserer(Id id, uint64_t) override {
        uint32_t i;
        if (!libres.empty()) {
            i = libres.back();
            libres.pop_back();
        } else {
            i = uint32_t(noeuds.size());
            noeuds.push_back({});
        }
        noeuds[i] = {id, NUL, NUL};
        index.emplace(id, i);
        accrocher(i);
    }
    void retirer(Id id) override {
        const auto it = index.find(id);
        const uint32_t i = it->second;
        index.erase(it);
        detacher(i);
        libres.push_back(i);
    }
    bool victime(const std::function<bool(Id)>& epingle, Id& v) override {
        for (uint32_t i = tete; i != NUL; i = noeuds[i].suiv)
            if (!epingle(noeuds[i].id)) {
                v = noeuds[i].id;
                return true;
            }
        return false;
    }
    std::vector<Id> ordre() const {
        std::vector<Id> o;
        for (uint32_t i = tete; i != NUL; i = noeuds[i].suiv) o.push_back(noeuds[i].id);
        return o;
    }
};

// Belady (MIN, offline optimum, simulator only): evict the non-pinned present id whose next use is
// the farthest; ties (same next group, or never again) go to the smallest (couche, expert). The
// instant is t = token * L + layer (trc-cache/src/politiques.rs:173-260). The next use is computed
// at access time, strictly after that access.
struct Belady final : Politique {
    std::unordered_map<Id, std::vector<uint64_t>> usages;
    std::vector<Id> presents;
    std::unordered_map<Id, size_t> rang;
    std::unordered_map<Id, uint64_t> prochain;

    explicit Belady(const Trace& tr) {
        const uint32_t L = tr.couches;
        for (uint32_t t = 0; t < tr.jetons; ++t)
            for (uint32_t c = 0; c < L; ++c) {
                const uint64_t instant = uint64_t(t) * L + c;
                const uint16_t* g = tr.groupe(t, c);
                for (uint32_t i = 0; i < tr.k; ++i) {
                    auto& v = usages[id_de(uint16_t(c), g[i])];
                    if (v.empty() || v.back() != instant) v.push_back(instant);
                }
            }
    }
    uint64_t prochain_apres(Id id, uint64_t t) const {
        const auto it = usages.find(id);
        if (it == usages.end()) return JAMAIS;
        const auto p = std::upper_bound(it->second.begin(), it->second.end(), t);
        return p == it->second.end() ? JAMAIS : *p;
    }
    void acceder(Id id, uint64_t t) override { prochain[id] = prochain_apres(id, t); }
    void inserer(Id id, uint64_t t) override {
        rang[id] = presents.size();
        presents.push_back(id);
        prochain[id] = prochain_apres(id, t);
    }
    void retirer(Id id) override {
        const size_t i = rang.at(id);
        rang.erase(id);
        presents[i] = presents.back();
        presents.pop_back();
        if (i < presents.size()) rang[presents[i]] = i;
        prochain.erase(id);
    }
    bool victime(const std::function<bool(Id)>& epingle, Id& v) override {
        bool trouve = false;
        uint64_t bp = 0;
        for (Id id : presents) {
            if (epingle(id)) continue;
            const uint64_t p = prochain.at(id);
            if (!trouve || p > bp || (p == bp && id < v)) {
                trouve = true;
                bp = p;
                v = id;
            }
        }
        return trouve;
    }
};

std::unique_ptr<Politique> politique(int sorte, const Trace* avenir) {
    switch (sorte) {
        case TRC_POLITIQUE_LRU: return std::make_unique<Lru>(false);
        case TRC_POLITIQUE_FIFO: return std::make_unique<Lru>(true);
        case TRC_POLITIQUE_BELADY:
            if (avenir == nullptr) return nullptr;
            return std::make_unique<Belady>(*avenir);
        default: return nullptr;
    }
}

}  // namespace

// ------------------------------------------------------------------------------- the cache

struct trc_trace {
    Trace t;
};

struct trc_cache {
    std::unique_ptr<Politique> vram, ram;
    std::vector<uint8_t> etats;  // TRC_CACHE_LIBRE / EN_VOL / PRESENT
    std::vector<Id> occupant;    // NUL when free
    std::unordered_map<Id, uint32_t> ou_vram;
    std::vector<uint32_t> libres_vram;
    std::vector<Id> occupant_tiede;
    std::unordered_map<Id, uint32_t> ou_ram;
    std::vector<uint32_t> libres_ram;
    std::vector<Id> epingles;
    std::vector<uint64_t> tailles;  // bytes read for an expert, [couche * experts + expert]
    uint16_t t_experts = 0;
    trc_compteurs_cache c{};

    bool epingle(Id id) const { return std::find(epingles.begin(), epingles.end(), id) != epingles.end(); }

    // A free slot, or the VRAM victim's (evicted here); NUL if every slot is pinned or in flight.
    uint32_t emplacement_pour_defaut() {
        if (!libres_vram.empty()) {
            const uint32_t s = libres_vram.back();
            libres_vram.pop_back();
            return s;
        }
        Id v;
        const bool ok = vram->victime(
            [&](Id id) {
                if (epingle(id)) return true;
                const auto it = ou_vram.find(id);
                return it != ou_vram.end() && etats[it->second] == TRC_CACHE_EN_VOL;
            },
            v);
        if (!ok) return NUL;
        vram->retirer(v);
        const uint32_t s = ou_vram.at(v);
        ou_vram.erase(v);
        occupant[s] = NUL;
        etats[s] = TRC_CACHE_LIBRE;
        c.evictions += 1;
        return s;
    }

    // A warm entry for a part read from disk; -1 without a RAM stage or when all are pinned.
    int32_t entree_tiede_pour(Id id, uint64_t t) {
        if (occupant_tiede.empty()) return -1;
        uint32_t r;
        if (!libres_ram.empty()) {
            r = libres_ram.back();
            libres_ram.pop_back();
        } else {
            Id v;
            if (!ram->victime([&](Id x) { return epingle(x); }, v)) return -1;
            ram->retirer(v);
            r = ou_ram.at(v);
            ou_ram.erase(v);
            occupant_tiede[r] = NUL;
            c.evictions_ram += 1;
        }
        ram->inserer(id, t);
        occupant_tiede[r] = id;
        ou_ram[id] = r;
        return int32_t(r);
    }

    uint64_t taille(Id id) const {
        if (tailles.empty()) return 0;
        const size_t i = size_t(id >> 16) * t_experts + (id & 0xFFFF);
        return i < tailles.size() ? tailles[i] : 0;
    }

    // Cache::demander (trc-cache/src/lib.rs:126-168): pins the layer's experts, then one decision
    // per expert in the given order. False when a miss finds neither a free slot nor a victim
    // (the caller sized the cache below the pinned experts): the cache is then unusable.
    bool demander(uint16_t couche, const uint16_t* experts, uint32_t n, uint64_t t, trc_decision* out) {
        for (uint32_t i = 0; i < n; ++i) {
            const Id id = id_de(couche, experts[i]);
            if (!epingle(id)) epingles.push_back(id);
        }
        for (uint32_t i = 0; i < n; ++i) {
            const Id id = id_de(couche, experts[i]);
            trc_decision& d = out[i];
            std::memset(&d, 0, sizeof(d));
            const auto hv = ou_vram.find(id);
            if (hv != ou_vram.end()) {
                vram->acceder(id, t);
                if (ou_ram.count(id)) ram->acceder(id, t);
                c.succes_vram += 1;
                d.sorte = TRC_DECISION_SUCCES;
                d.emplacement = hv->second;
                d.tiede = -1;
                continue;
            }
            const uint32_t s = emplacement_pour_defaut();
            if (s == NUL) return false;
            vram->inserer(id, t);
            etats[s] = TRC_CACHE_EN_VOL;
            occupant[s] = id;
            ou_vram[id] = s;
            const uint64_t octets = taille(id);
            c.octets_copies += octets;
            d.emplacement = s;
            const auto hr = ou_ram.find(id);
            if (hr != ou_ram.end()) {
                ram->acceder(id, t);
                c.succes_ram += 1;
                d.sorte = TRC_DECISION_DEFAUT_RAM;
                d.tiede = int32_t(hr->second);
            } else {
                c.defauts_disque += 1;
                c.octets_disque += octets;
                d.sorte = TRC_DECISION_DEFAUT_DISQUE;
                d.tiede = entree_tiede_pour(id, t);
            }
        }
        return true;
    }

    void liberer(uint16_t couche) {
        epingles.erase(std::remove_if(epingles.begin(), epingles.end(), [&](Id id) { return (id >> 16) == couche; }),
                       epingles.end());
    }
};

namespace {

trc_cache* nouveau_cache(uint32_t emplacements, uint32_t tiedes, std::unique_ptr<Politique> v,
                         std::unique_ptr<Politique> r) {
    auto c = std::make_unique<trc_cache>();
    c->vram = std::move(v);
    c->ram = std::move(r);
    c->etats.assign(emplacements, TRC_CACHE_LIBRE);
    c->occupant.assign(emplacements, NUL);
    for (uint32_t s = emplacements; s-- > 0;) c->libres_vram.push_back(s);  // served 0, 1, 2, ...
    c->occupant_tiede.assign(tiedes, NUL);
    for (uint32_t s = tiedes; s-- > 0;) c->libres_ram.push_back(s);
    return c.release();
}

// Trace::depuis_texte (trc-cache/src/trace.rs:51-130): one token per line, layers separated by
// '|', experts by blanks; '#' comments; "E=<n>" declares the experts per layer (else the largest
// id + 1). Refused, with the line: a different layer count, a layer without k experts, an
// unreadable id or E, an id outside [0, E), no token line.
int lire_trace(const char* texte, uint64_t n, Trace& tr, std::string& commentaires) {
    int e_declare = -1;
    uint32_t couches = 0, k = 0, jetons = 0;
    uint64_t p = 0;
    uint32_t numero = 0;
    auto ligne_err = [&](const std::string& raison) {
        trc::derniere_erreur() = "trace, ligne " + std::to_string(numero) + " : " + raison;
        return TRC_TRACE_LIGNE;
    };
    while (p < n) {
        uint64_t q = p;
        while (q < n && texte[q] != '\n') ++q;
        std::string ligne(texte + p, texte + q);
        p = q + 1;
        ++numero;
        const auto deb = ligne.find_first_not_of(" \t\r");
        if (deb == std::string::npos) continue;
        const auto fin = ligne.find_last_not_of(" \t\r");
        ligne = ligne.substr(deb, fin - deb + 1);
        if (ligne[0] == '#') {
            std::string c = ligne.substr(1);
            const auto d2 = c.find_first_not_of(" \t");
            commentaires += (d2 == std::string::npos ? "" : c.substr(d2)) + "\n";
            continue;
        }
        if (ligne.compare(0, 2, "E=") == 0) {
            char* f = nullptr;
            const std::string v = ligne.substr(2);
            const long e = std::strtol(v.c_str(), &f, 10);
            if (v.empty() || f == v.c_str() || *f != '\0' || e < 0 || e > 65535)
                return ligne_err("« E= » illisible : " + v);
            if (e == 0) return ligne_err("E = 0");
            e_declare = int(e);
            continue;
        }
        std::vector<std::string> parts;
        size_t a = 0;
        for (size_t b; (b = ligne.find('|', a)) != std::string::npos; a = b + 1) parts.push_back(ligne.substr(a, b - a));
        parts.push_back(ligne.substr(a));
        if (jetons == 0) couches = uint32_t(parts.size());
        else if (parts.size() != couches)
            return ligne_err(std::to_string(parts.size()) + " couches au lieu de " + std::to_string(couches));
        for (uint32_t l = 0; l < parts.size(); ++l) {
            const size_t avant = tr.choix.size();
            const char* s = parts[l].c_str();
            while (*s) {
                while (*s == ' ' || *s == '\t' || *s == '\r') ++s;
                if (!*s) break;
                const char* m = s;
                while (*s && *s != ' ' && *s != '\t' && *s != '\r') ++s;
                const std::string mot(m, s);
                char* f = nullptr;
                const unsigned long x = std::strtoul(mot.c_str(), &f, 10);
                if (*f != '\0' || mot[0] == '-' || mot[0] == '+' || x > 65535)
                    return ligne_err("identifiant d'expert illisible : " + mot);
                tr.choix.push_back(uint16_t(x));
            }
            const uint32_t nc = uint32_t(tr.choix.size() - avant);
            if (jetons == 0 && l == 0) {
                k = nc;
                if (k == 0) return ligne_err("couche vide");
            } else if (nc != k) {
                return ligne_err("couche " + std::to_string(l) + " : " + std::to_string(nc) + " experts au lieu de " +
                                 std::to_string(k));
            }
        }
        ++jetons;
    }
    if (jetons == 0) {
        trc::derniere_erreur() = "trace vide (aucune ligne de jeton)";
        return TRC_TRACE_VIDE;
    }
    const uint16_t mx = *std::max_element(tr.choix.begin(), tr.choix.end());
    uint32_t experts;
    if (e_declare >= 0) {
        if (mx >= e_declare) {
            trc::derniere_erreur() =
                "trace : expert " + std::to_string(mx) + " hors de [0, " + std::to_string(e_declare) + ")";
            return TRC_TRACE_HORS_BORNES;
        }
        experts = uint32_t(e_declare);
    } else {
        if (mx == 65535) {
            trc::derniere_erreur() = "trace : expert 65535 hors de [0, 65535)";
            return TRC_TRACE_HORS_BORNES;
        }
        experts = mx + 1u;
    }
    if (couches > 65535 || k > 65535) {
        numero = 0;
        return ligne_err("dimensions hors de u16");
    }
    tr.experts = uint16_t(experts);
    tr.couches = uint16_t(couches);
    tr.k = uint16_t(k);
    tr.jetons = jetons;
    return TRC_OK;
}

}  // namespace

extern "C" {

int trc_trace_depuis_texte(const char* texte, uint64_t n, trc_trace** sortie) {
    if (texte == nullptr || sortie == nullptr) return trc::usage("pointeur nul");
    *sortie = nullptr;
    auto t = std::make_unique<trc_trace>();
    std::string com;
    const int r = lire_trace(texte, n, t->t, com);
    if (r == TRC_OK) *sortie = t.release();
    return r;
}

int trc_trace_creer(uint16_t experts, uint16_t couches, uint16_t k, uint32_t jetons, const uint16_t* choix,
                    trc_trace** sortie) {
    if (sortie == nullptr || (choix == nullptr && jetons)) return trc::usage("pointeur nul");
    *sortie = nullptr;
    if (experts == 0 || couches == 0 || k == 0 || jetons == 0) return trc::usage("trace : dimensions nulles");
    const size_t n = size_t(jetons) * couches * k;
    for (size_t i = 0; i < n; ++i)
        if (choix[i] >= experts) return trc::usage("trace : expert %u hors de [0, %u)", choix[i], experts);
    auto t = std::make_unique<trc_trace>();
    t->t.experts = experts;
    t->t.couches = couches;
    t->t.k = k;
    t->t.jetons = jetons;
    t->t.choix.assign(choix, choix + n);
    *sortie = t.release();
    return TRC_OK;
}

void trc_trace_dimensions(const trc_trace* t, uint32_t dims[4]) {
    dims[0] = t->t.experts;
    dims[1] = t->t.couches;
    dims[2] = t->t.k;
    dims[3] = t->t.jetons;
}

const uint16_t* trc_trace_groupe(const trc_trace* t, uint32_t jeton, uint32_t couche) {
    if (jeton >= t->t.jetons || couche >= t->t.couches) return nullptr;
    return t->t.groupe(jeton, couche);
}

void trc_trace_liberer(trc_trace* t) { delete t; }

int trc_cache_creer(uint32_t emplacements, uint32_t tiedes, int politique_vram, int politique_ram,
                    const trc_trace* avenir, trc_cache** sortie) {
    if (sortie == nullptr) return trc::usage("pointeur nul");
    *sortie = nullptr;
    auto v = politique(politique_vram, avenir ? &avenir->t : nullptr);
    auto r = politique(politique_ram, avenir ? &avenir->t : nullptr);
    if (!v || !r) return trc::usage("politique inconnue, ou Belady sans la trace de l'avenir");
    *sortie = nouveau_cache(emplacements, tiedes, std::move(v), std::move(r));
    return TRC_OK;
}

void trc_cache_detruire(trc_cache* c) { delete c; }

int trc_cache_fixer_tailles(trc_cache* c, uint16_t couches, uint16_t experts, const uint64_t* tailles) {
    if (c == nullptr || tailles == nullptr || couches == 0 || experts == 0) return trc::usage("arguments faux");
    c->t_experts = experts;
    c->tailles.assign(tailles, tailles + size_t(couches) * experts);
    return TRC_OK;
}

int trc_cache_demander(trc_cache* c, uint16_t couche, const uint16_t* experts, uint32_t n, uint64_t t,
                       trc_decision* decisions) {
    if (c == nullptr || (n && (experts == nullptr || decisions == nullptr))) return trc::usage("pointeur nul");
    if (!c->demander(couche, experts, n, t, decisions))
        return trc::usage("cache : aucun emplacement VRAM libre ni evincable (%zu emplacements, %zu experts "
                          "epingles) : il faut emplacements >= experts epingles a la fois",
                          c->etats.size(), c->epingles.size());
    return TRC_OK;
}

int trc_cache_pret(trc_cache* c, uint32_t emplacement) {
    if (c == nullptr || emplacement >= c->etats.size()) return trc::usage("emplacement hors du cache");
    if (c->etats[emplacement] != TRC_CACHE_EN_VOL)
        return trc::usage("cache : pret(%u) sur un emplacement %s", emplacement,
                          c->etats[emplacement] == TRC_CACHE_LIBRE ? "libre" : "present");
    c->etats[emplacement] = TRC_CACHE_PRESENT;
    return TRC_OK;
}

void trc_cache_liberer_couche(trc_cache* c, uint16_t couche) { c->liberer(couche); }

trc_compteurs_cache trc_cache_compteurs(const trc_cache* c) { return c->c; }

int trc_cache_etat(const trc_cache* c, uint32_t emplacement) {
    return emplacement < c->etats.size() ? c->etats[emplacement] : -1;
}

int64_t trc_cache_occupant(const trc_cache* c, uint32_t emplacement) {
    if (emplacement >= c->occupant.size() || c->occupant[emplacement] == NUL) return -1;
    return c->occupant[emplacement];
}

int64_t trc_cache_emplacement_de(const trc_cache* c, uint16_t couche, uint16_t expert) {
    const auto it = c->ou_vram.find(id_de(couche, expert));
    return it == c->ou_vram.end() ? -1 : int64_t(it->second);
}

int64_t trc_cache_tiede_de(const trc_cache* c, uint16_t couche, uint16_t expert) {
    const auto it = c->ou_ram.find(id_de(couche, expert));
    return it == c->ou_ram.end() ? -1 : int64_t(it->second);
}

uint32_t trc_cache_epingles(const trc_cache* c, uint32_t* ids, uint32_t max) {
    const uint32_t n = uint32_t(c->epingles.size());
    for (uint32_t i = 0; i < n && i < max; ++i) ids[i] = c->epingles[i];
    return n;
}

uint32_t trc_cache_ordre_vram(const trc_cache* c, uint32_t* ids, uint32_t max) {
    const Lru* l = dynamic_cast<const Lru*>(c->vram.get());
    if (l == nullptr) return 0;
    const auto o = l->ordre();
    for (uint32_t i = 0; i < o.size() && i < max; ++i) ids[i] = o[i];
    return uint32_t(o.size());
}

// rejouer_dans (trc-cache/src/lib.rs:290-309): for each token, each layer in compute order,
// demander, pret on every miss, then liberer; the policies' instant is t = token * L + layer.
int trc_cache_rejouer_dans(trc_cache* c, const trc_trace* tr, trc_compteurs_cache* sortie) {
    if (c == nullptr || tr == nullptr) return trc::usage("pointeur nul");
    const Trace& T = tr->t;
    std::vector<trc_decision> d(T.k);
    for (uint32_t t = 0; t < T.jetons; ++t)
        for (uint32_t l = 0; l < T.couches; ++l) {
            const int r = trc_cache_demander(c, uint16_t(l), T.groupe(t, l), T.k, uint64_t(t) * T.couches + l, d.data());
            if (r != TRC_OK) return r;
            for (const trc_decision& x : d)
                if (x.sorte != TRC_DECISION_SUCCES) c->etats[x.emplacement] = TRC_CACHE_PRESENT;
            c->liberer(uint16_t(l));
        }
    if (sortie) *sortie = c->c;
    return TRC_OK;
}

// rejouer (trc-cache/src/lib.rs:282-286): the simulator, on a fresh cache (counts in accesses).
int trc_cache_rejouer(const trc_trace* tr, uint32_t emplacements, uint32_t tiedes, int politique_vram,
                      int politique_ram, trc_compteurs_cache* sortie) {
    trc_cache* c = nullptr;
    int r = trc_cache_creer(emplacements, tiedes, politique_vram, politique_ram, tr, &c);
    if (r != TRC_OK) return r;
    r = trc_cache_rejouer_dans(c, tr, sortie);
    delete c;
    return r;
}

}  // extern "C"
