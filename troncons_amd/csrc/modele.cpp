// modele.cpp — native driver of one decode step (trc_modele::Modele, moteur/crates/trc-modele/
// src/lib.rs:476-568): embedding row, then per layer the attention half (debut_couche: RMSNorm,
// Q/K/V Q8_0 GEMVs, YaRN, f16 KV write, sink attention, output projection, residual add,
// post-attention RMSNorm) and the MoE half (the fused compressed layer: router, top-k, the k
// rANS-decoded experts, SwiGLU, the ordered combine into the residual), then the output head
// (RMSNorm, Q8_0 logits, argmax). Every launch is one of this library's C-ABI entry points, issued
// from here in the reference's order: one call per token from the host, no host synchronisation.
//
// The caller owns the weights, the KV caches and the layers' mounted directories (device views);
// the driver owns nothing but a copy of those views and the workspace view it is given.
#include <hip/hip_runtime.h>

#include <cstring>
#include <new>
#include <vector>

#include "../../include/troncons_hip.h"
#include "erreurs.hpp"
#include "passe.hpp"

struct trc_modele {
    trc_hyper h;
    std::vector<trc_couche_modele> c;
    trc_vue emb, norme_sortie, sortie;
    // workspace pieces
    trc_vue x, hh, h2, q, k, v, a, o, idx, pw, controle, moe, z, jeton, table;
    int64_t position_table = -1;  // the position whose rotation table is in `table` (-1: none yet)
};

namespace {

uint64_t al(uint64_t x) { return (x + 255u) & ~uint64_t(255); }

uint32_t anneau(const trc_hyper& h, uint32_t l) { return l % 2u == 0u ? h.fenetre : 0u; }

// Cuts the workspace into the step's buffers (sizes in order of trc_modele_taille_travail).
struct Decoupe {
    uint64_t p;
    trc_vue prendre(uint64_t octets) {
        trc_vue v{p, octets};
        p += al(octets);
        return v;
    }
};

uint64_t taille_moe(const trc_hyper& h) {
    return trc_taille_travail_couche_moe(&h.dims, h.experts, h.actifs, h.n_codes);
}

uint64_t taille_travail(const trc_hyper& h) {
    const uint64_t d = h.d, dq = uint64_t(h.tetes) * 64, dkv = uint64_t(h.tetes_kv) * 64;
    return al(4 * d) * 3 + al(4 * dq) * 2 + al(4 * dkv) * 2 + al(4 * d) + al(4 * 8) * 2 + al(16) + al(taille_moe(h)) +
           al(4ull * h.vocab) + al(4) + al(16 * 32);
}

int verifier_hyper(const trc_hyper* h) {
    if (h == nullptr) return trc::usage("hyperparametres absents");
    if (h->couches == 0 || h->d == 0 || h->d % 32 != 0) return trc::usage("%u couches de dimension %u", h->couches, h->d);
    if (h->tetes == 0 || h->tetes_kv == 0 || h->tetes % h->tetes_kv != 0)
        return trc::usage("tetes %u / %u", h->tetes, h->tetes_kv);
    if (h->rope.dim_tete != 64) return trc::usage("dimension de tete %u (64 seulement)", h->rope.dim_tete);
    if (h->contexte == 0 || h->contexte > TRC_ATTENTION_POSITIONS_MAX)
        return trc::usage("contexte de %u positions (1 a %u)", h->contexte, TRC_ATTENTION_POSITIONS_MAX);
    if (h->vocab == 0) return trc::usage("vocabulaire vide");
    if (taille_moe(*h) == 0) return trc::usage("couche MoE refusee (formes, k %u, experts %u)", h->actifs, h->experts);
    if (h->dims.colonnes[0] != h->d || h->dims.lignes[2] != h->d)
        return trc::usage("experts %u -> %u incompatibles avec d = %u", h->dims.colonnes[0], h->dims.lignes[2], h->d);
    return TRC_OK;
}

}  // namespace

extern "C" uint64_t trc_modele_taille_travail(const trc_hyper* h) {
    if (verifier_hyper(h) != TRC_OK) return 0;
    return taille_travail(*h);
}

extern "C" int trc_modele_creer(const trc_hyper* h, const trc_couche_modele* couches, trc_vue enchassement,
                                trc_vue norme_sortie, trc_vue sortie, trc_vue travail, trc_modele** m) {
    if (m == nullptr) return trc::usage("sortie nulle");
    *m = nullptr;
    int r = verifier_hyper(h);
    if (r != TRC_OK) return r;
    if (couches == nullptr) return trc::usage("couches absentes");
    const uint64_t besoin = taille_travail(*h);
    TRC_VERIFIER(travail.adresse && travail.adresse % 256 == 0 && travail.octets >= besoin,
                 "travail de %llu o, %llu o demandes (aligne sur 256)", (unsigned long long)travail.octets,
                 (unsigned long long)besoin);
    const uint64_t dkv = uint64_t(h->tetes_kv) * 64;
    for (uint32_t l = 0; l < h->couches; ++l) {
        const uint64_t cases = anneau(*h, l) ? anneau(*h, l) : h->contexte;
        TRC_VERIFIER(couches[l].cache_k.octets >= 2 * cases * dkv && couches[l].cache_v.octets >= 2 * cases * dkv,
                     "couche %u : cache de %llu o pour %llu cases", l, (unsigned long long)couches[l].cache_k.octets,
                     (unsigned long long)cases);
    }
    trc_modele* n = new (std::nothrow) trc_modele;
    if (n == nullptr) return trc::usage("memoire hote epuisee");
    n->h = *h;
    n->c.assign(couches, couches + h->couches);
    n->emb = enchassement;
    n->norme_sortie = norme_sortie;
    n->sortie = sortie;
    const uint64_t d = h->d, dq = uint64_t(h->tetes) * 64;
    Decoupe t{travail.adresse};
    n->x = t.prendre(4 * d);
    n->hh = t.prendre(4 * d);
    n->h2 = t.prendre(4 * d);
    n->q = t.prendre(4 * dq);
    n->a = t.prendre(4 * dq);
    n->k = t.prendre(4 * dkv);
    n->v = t.prendre(4 * dkv);
    n->o = t.prendre(4 * d);
    n->idx = t.prendre(4 * 8);
    n->pw = t.prendre(4 * 8);
    n->controle = t.prendre(16);
    n->moe = t.prendre(taille_moe(*h));
    n->z = t.prendre(4ull * h->vocab);
    n->jeton = t.prendre(4);
    n->table = t.prendre(16 * 32);
    *m = n;
    return TRC_OK;
}

extern "C" void trc_modele_detruire(trc_modele* m) { delete m; }

extern "C" int trc_modele_vues(const trc_modele* m, trc_vue* x, trc_vue* logits, trc_vue* jeton, trc_vue* indices,
                               trc_vue* controle) {
    if (m == nullptr) return trc::usage("modele nul");
    if (x) *x = m->x;
    if (logits) *logits = m->z;
    if (jeton) *jeton = m->jeton;
    if (indices) *indices = m->idx;
    if (controle) *controle = m->controle;
    return TRC_OK;
}

// Modele::enchasser (lib.rs:481-487).
extern "C" int trc_modele_enchasser(trc_modele* m, uint32_t jeton, void* flux) {
    if (m == nullptr) return trc::usage("modele nul");
    TRC_VERIFIER(jeton < m->h.vocab, "jeton %u hors du vocabulaire de %u", jeton, m->h.vocab);
    return trc_ligne_q8_0(m->emb, jeton, m->h.d, m->x, flux);
}

// Modele::debut_couche up to the post-attention norm (lib.rs:498-521), then the fused MoE half.
// The norm, the three projections, the rotation and the KV write go out as one launch, the output
// projection and the residual add as another, with the values of the separate kernels.
extern "C" int trc_modele_couche(trc_modele* m, uint32_t l, uint32_t position, void* flux) {
    if (m == nullptr) return trc::usage("modele nul");
    const trc_hyper& h = m->h;
    TRC_VERIFIER(l < h.couches, "couche %u sur %u", l, h.couches);
    TRC_VERIFIER(position < h.contexte, "position %u au-dela du contexte de %u positions", position, h.contexte);
    const trc_couche_modele& c = m->c[l];
    const uint32_t d = h.d, dq = h.tetes * 64, dkv = h.tetes_kv * 64, an = anneau(h, l);
    int r;
#define TRC_ETAPE(appel)          \
    do {                          \
        r = (appel);              \
        if (r != TRC_OK) return r; \
    } while (0)
    // the rotation coefficients once per position (every layer shares them), then rmsnorm, the
    // q, k, v GEMVs, rope_yarn and ecrire_kv in one launch
    if (m->position_table != int64_t(position)) {
        TRC_ETAPE(trc::lancer_table_rope(&h.rope, position, m->table, flux));
        m->position_table = position;
    }
    const trc_vue w[3] = {c.wq, c.wk, c.wv}, b[3] = {c.bq, c.bk, c.bv}, y[3] = {m->q, m->k, m->v};
    const uint32_t lignes[3] = {dq, dkv, dkv};
    TRC_ETAPE(trc::lancer_qkv_q8_0(m->x, c.attn_norm, h.eps, d, w, b, y, lignes, c.cache_k, c.cache_v, m->table,
                                   an ? position % an : position, flux));
    trc_params_attention pa;
    pa.tetes = h.tetes;
    pa.tetes_kv = h.tetes_kv;
    pa.dim_tete = 64;
    pa.fin = position + 1;
    pa.debut = an ? (pa.fin > an ? pa.fin - an : 0u) : 0u;
    pa.anneau = an;
    pa.echelle = 0.125f;
    pa.reserve = 0;
    TRC_ETAPE(trc_attention(m->q, c.cache_k, c.cache_v, c.puits, m->a, &pa, flux));
    // the output projection adds itself into the residual (gemv_q8_0 + combiner)
    TRC_ETAPE(trc::lancer_gemv_q8_0_residu(c.wo, m->a, c.bo, m->x, d, dq, flux));
    // the post-attention norm goes into the MoE router's launch, which leaves h2 for the later passes
    TRC_ETAPE(trc::lancer_couche_moe_normee(c.repertoire, h.experts, c.luts, &h.dims, c.routeur, c.routeur_biais,
                                            c.post_norm, h.eps, m->h2, h.actifs, m->x, m->idx, m->pw, m->controle,
                                            m->moe, h.n_delta, h.n_codes, flux));
#undef TRC_ETAPE
    return TRC_OK;
}

// Modele::sortie (lib.rs:557-568).
extern "C" int trc_modele_sortie(trc_modele* m, void* flux) {
    if (m == nullptr) return trc::usage("modele nul");
    const trc_hyper& h = m->h;
    int r = trc_rmsnorm(m->x, m->norme_sortie, m->hh, h.d, 1, h.eps, flux);
    if (r == TRC_OK) r = trc_gemv_q8_0(m->sortie, m->hh, trc_vue{0, 0}, m->z, h.vocab, h.d, flux);
    if (r == TRC_OK) r = trc_argmax(m->z, h.vocab, m->jeton, flux);
    return r;
}

// One decode step of `jeton` at `position` through every layer and the head (asynchronous).
extern "C" int trc_modele_pas(trc_modele* m, uint32_t jeton, uint32_t position, void* flux) {
    int r = trc_modele_enchasser(m, jeton, flux);
    for (uint32_t l = 0; r == TRC_OK && l < m->h.couches; ++l) r = trc_modele_couche(m, l, position, flux);
    if (r == TRC_OK) r = trc_modele_sortie(m, flux);
    return r;
}
