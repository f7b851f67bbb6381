// diffusion.cpp — the streamed MoE layer on the fused path (host C++ over HIP): the experts' coded
// parts stay in pinned host memory; per layer and token only the k chosen ones cross the host link,
// and each is decoded inside its fused MLP straight from its arrival buffer (no decoded slot).
//
// Per layer (the expert part of the reference's Moteur::pas with every part in RAM,
// moteur/crates/trc-ordo/src/lib.rs:1054-1128 and 1328-1370, on the fused kernels):
//   1. router on the caller's compute stream (gemv_f32 + routeur_topk), the kernel writing the k
//      indices and a sequence word into a mapped host mailbox; the host waits for the router's event
//      and reads the mailbox: the layer's one device -> host wait;
//   2. the k parts copied on the engine's copy stream into one of two sets of k device arrival
//      buffers (the set of layer n % 2, so that layer n's copies overlap nothing of layer n - 1 they
//      would overwrite: the copy stream first waits for the event recorded after the last layer that
//      used the set), one event per copy;
//   3. on the compute stream, expert q waits for its copy's event, then trc_expert_fusionne (decode
//      in registers, gate/up GEMVs, SwiGLU, down GEMV) writes its output row; copy q + 1 lands
//      meanwhile;
//   4. trc_combiner adds the weighted outputs to the residual in expert order.
// Every launch is the library's own entry point, so the residuals are those of the resident layer
// step bit for bit (the same fused arithmetic; the tests check it).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "commun.hpp"
#include "erreurs.hpp"

namespace {

using horloge = std::chrono::steady_clock;

#define TRC_HIP(appel)                                              \
    do {                                                            \
        const hipError_t e_ = (appel);                              \
        if (e_ != hipSuccess) return ::trc::erreur_hip(#appel, e_); \
    } while (0)

#define TRC_OK_OU_RENDRE(expr)       \
    do {                             \
        const int r_ = (expr);       \
        if (r_ != TRC_OK) return r_; \
    } while (0)

trc_vue vue(const void* p, uint64_t n) { return trc_vue{uint64_t(reinterpret_cast<uintptr_t>(p)), n}; }

}  // namespace

struct trc_diffusion {
    struct Couche {
        const uint8_t* parties = nullptr;
        std::vector<uint64_t> decalages, tailles;
        trc_vue luts{0, 0}, routeur{0, 0};
    };
    std::vector<Couche> couches;
    uint32_t E = 0, k = 0, C = 0, D = 0, n_delta = 0, n_codes = 0;
    trc_dims_expert dims{};
    uint64_t t_max = 0;        // largest part of any layer (arrival buffer size, 256-aligned)
    uint8_t* arrivees = nullptr;  // [2][k][t_max]
    float* logits = nullptr;
    uint32_t* idx = nullptr;
    float* poids = nullptr;
    float* sorties = nullptr;  // [k][D]
    uint8_t* travail = nullptr;
    uint64_t octets_travail = 0;
    uint32_t* controle = nullptr;  // u32[4], zeroed at creation
    uint32_t* boite = nullptr;     // mapped host mailbox
    uint32_t* boite_carte = nullptr;
    hipStream_t copie = nullptr;
    hipEvent_t ev_routeur = nullptr;
    hipEvent_t ev_arr[2][8] = {};
    hipEvent_t ev_libre[2] = {};
    bool libre_enregistre[2] = {false, false};
    uint32_t sequence = 0;
    uint64_t n_couches_faites = 0;
    trc_stats_diffusion st{};
    // fail-stop, as the reference engine (which panics): after a layer failed part-way, copies and
    // launches of it may still be in flight over the arrival buffers, so later layers are refused
    bool en_echec = false;

    ~trc_diffusion() {
        for (auto& v : ev_arr)
            for (hipEvent_t e : v)
                if (e) (void)hipEventDestroy(e);
        for (hipEvent_t e : ev_libre)
            if (e) (void)hipEventDestroy(e);
        if (ev_routeur) (void)hipEventDestroy(ev_routeur);
        if (copie) (void)hipStreamDestroy(copie);
        if (boite) (void)hipHostFree(boite);
        for (void* p : {static_cast<void*>(arrivees), static_cast<void*>(logits), static_cast<void*>(idx),
                        static_cast<void*>(poids), static_cast<void*>(sorties), static_cast<void*>(travail),
                        static_cast<void*>(controle)})
            if (p) (void)hipFree(p);
    }

    int couche(uint32_t l, const trc_vue& x, const trc_vue& residu, void* flux, uint32_t* choisis) {
        const hipStream_t fl = reinterpret_cast<hipStream_t>(flux);
        const Couche& c = couches[l];
        // 1. router and mailbox
        sequence = sequence + 1 == 0 ? 1 : sequence + 1;
        const uint32_t seq = sequence;
        TRC_OK_OU_RENDRE(trc_gemv_f32(c.routeur, x, trc_vue{0, 0}, vue(logits, 4ull * E), E, C, flux));
        TRC_OK_OU_RENDRE(trc_routeur_topk(vue(logits, 4ull * E), E, k, vue(idx, 64), vue(poids, 64),
                                          uint64_t(reinterpret_cast<uintptr_t>(boite_carte)), seq, flux));
        TRC_HIP(hipEventRecord(ev_routeur, fl));
        const auto t0 = horloge::now();
        TRC_HIP(hipEventSynchronize(ev_routeur));
        st.us_attente_routeur += std::chrono::duration<double, std::micro>(horloge::now() - t0).count();
        const volatile uint32_t* bv = boite;
        if (bv[0] != seq) return trc::usage("couche %u : boite a la sequence %u, %u attendue", l, bv[0], seq);
        uint32_t experts[8];
        for (uint32_t i = 0; i < k; ++i) {
            experts[i] = bv[1 + i];
            if (experts[i] >= E) return trc::usage("couche %u : expert %u hors de [0, %u)", l, experts[i], E);
            if (choisis) choisis[i] = experts[i];
        }
        // 2. copies into the set of this layer, once the set's previous readers are done
        const uint32_t s = uint32_t(n_couches_faites & 1u);
        if (libre_enregistre[s]) TRC_HIP(hipStreamWaitEvent(copie, ev_libre[s], 0));
        for (uint32_t q = 0; q < k; ++q) {
            const uint32_t e = experts[q];
            uint8_t* dst = arrivees + (uint64_t(s) * k + q) * t_max;
            TRC_HIP(hipMemcpyAsync(dst, c.parties + c.decalages[e], c.tailles[e], hipMemcpyHostToDevice, copie));
            TRC_HIP(hipEventRecord(ev_arr[s][q], copie));
            st.octets_copies += c.tailles[e];
        }
        // 3. each expert once its part has landed
        for (uint32_t q = 0; q < k; ++q) {
            TRC_HIP(hipStreamWaitEvent(fl, ev_arr[s][q], 0));
            uint8_t* src = arrivees + (uint64_t(s) * k + q) * t_max;
            TRC_OK_OU_RENDRE(trc_expert_fusionne(vue(src, c.tailles[experts[q]]), c.luts, &dims, x,
                                                 vue(sorties + uint64_t(q) * D, 4ull * D), vue(controle, 16),
                                                 vue(travail, octets_travail), n_delta, n_codes, flux));
        }
        // 4. the ordered combine
        TRC_OK_OU_RENDRE(trc_combiner(residu, vue(sorties, 4ull * k * D), D, vue(poids, 4ull * k), k, D, flux));
        TRC_HIP(hipEventRecord(ev_libre[s], fl));
        libre_enregistre[s] = true;
        n_couches_faites += 1;
        st.couches += 1;
        return TRC_OK;
    }
};

extern "C" int trc_diffusion_creer(const trc_couche_hote* couches, uint32_t n_couches, uint32_t experts, uint32_t k,
                                   const trc_dims_expert* dims, uint32_t n_delta, uint32_t n_codes,
                                   trc_diffusion** sortie) {
    if (sortie == nullptr) return trc::usage("sortie nulle");
    *sortie = nullptr;
    if (couches == nullptr || n_couches == 0) return trc::usage("aucune couche");
    if (dims == nullptr) return trc::usage("dims absent");
    int r = trc_dims_verifier(dims);
    if (r != TRC_OK) return r;
    if (experts == 0 || experts > 256 || k == 0 || k > 8 || k > experts)
        return trc::usage("top-%u sur %u experts", k, experts);
    if (dims->colonnes[0] != dims->colonnes[1] || dims->lignes[0] != dims->lignes[1] ||
        dims->colonnes[2] != dims->lignes[0] || dims->lignes[2] != dims->colonnes[0])
        return trc::usage("gate, up et down incompatibles");
    const uint64_t tr = trc_taille_travail_expert_fusionne(dims, n_codes);
    if (tr == 0) return trc::usage("forme ou N refuses par le chemin fusionne");
    auto m = std::make_unique<trc_diffusion>();
    m->E = experts;
    m->k = k;
    m->C = dims->colonnes[0];
    m->D = dims->lignes[2];
    m->n_delta = n_delta;
    m->n_codes = n_codes;
    m->dims = *dims;
    m->octets_travail = tr;
    for (uint32_t l = 0; l < n_couches; ++l) {
        const trc_couche_hote& h = couches[l];
        if (h.parties == nullptr || h.decalages == nullptr || h.tailles == nullptr)
            return trc::usage("couche %u : parties absentes", l);
        if (h.luts.adresse == 0 || h.luts.octets < uint64_t(trc::LUTS_PAR_COUCHE) * 4)
            return trc::usage("couche %u : LUT trop courtes", l);
        if (h.routeur.adresse == 0 || h.routeur.octets < 4ull * experts * m->C || h.routeur.adresse % 16 != 0)
            return trc::usage("couche %u : routeur f32 trop court ou non aligne sur 16", l);
        trc_diffusion::Couche c;
        c.parties = static_cast<const uint8_t*>(h.parties);
        c.decalages.assign(h.decalages, h.decalages + experts);
        c.tailles.assign(h.tailles, h.tailles + experts);
        for (uint32_t e = 0; e < experts; ++e) {
            if (c.tailles[e] < 64 || (reinterpret_cast<uintptr_t>(c.parties) + c.decalages[e]) % 16 != 0)
                return trc::usage("couche %u, expert %u : partie trop courte ou non alignee sur 16", l, e);
            m->t_max = std::max(m->t_max, (c.tailles[e] + 255) / 256 * 256);
        }
        c.luts = h.luts;
        c.routeur = h.routeur;
        m->couches.push_back(std::move(c));
    }
    TRC_HIP(hipMalloc(&m->arrivees, 2ull * k * m->t_max));
    TRC_HIP(hipMalloc(&m->logits, 4ull * experts));
    TRC_HIP(hipMalloc(&m->idx, 64));
    TRC_HIP(hipMalloc(&m->poids, 64));
    TRC_HIP(hipMalloc(&m->sorties, 4ull * k * m->D));
    TRC_HIP(hipMalloc(&m->travail, m->octets_travail));
    TRC_HIP(hipMalloc(&m->controle, 16));
    TRC_HIP(hipMemset(m->controle, 0, 16));
    TRC_HIP(hipHostMalloc(&m->boite, 256, hipHostMallocMapped));
    std::memset(m->boite, 0, 256);
    TRC_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&m->boite_carte), m->boite, 0));
    TRC_HIP(hipStreamCreateWithFlags(&m->copie, hipStreamNonBlocking));
    TRC_HIP(hipEventCreateWithFlags(&m->ev_routeur, hipEventDisableTiming));
    for (auto& v : m->ev_arr)
        for (uint32_t q = 0; q < k; ++q) TRC_HIP(hipEventCreateWithFlags(&v[q], hipEventDisableTiming));
    for (hipEvent_t& e : m->ev_libre) TRC_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    TRC_HIP(hipDeviceSynchronize());
    *sortie = m.release();
    return TRC_OK;
}

extern "C" void trc_diffusion_detruire(trc_diffusion* m) {
    if (m == nullptr) return;
    (void)hipDeviceSynchronize();
    delete m;
}

extern "C" int trc_diffusion_couche(trc_diffusion* m, uint32_t couche, trc_vue x, trc_vue residu, void* flux,
                                    uint32_t* choisis) {
    if (m == nullptr) return trc::usage("moteur nul");
    if (m->en_echec) return trc::usage("moteur arrete par une erreur precedente");
    if (couche >= m->couches.size()) return trc::usage("couche %u sur %zu", couche, m->couches.size());
    if (x.adresse == 0 || x.octets < 4ull * m->C || x.adresse % 16 != 0) return trc::usage("x trop court ou non aligne");
    if (residu.adresse == 0 || residu.octets < 4ull * m->D) return trc::usage("residu trop court");
    const int r = m->couche(couche, x, residu, flux, choisis);
    if (r != TRC_OK) {
        // drain what the failed layer queued, keep the error's message
        const std::string message = trc_derniere_erreur();
        (void)hipStreamSynchronize(m->copie);
        (void)hipStreamSynchronize(reinterpret_cast<hipStream_t>(flux));
        m->en_echec = true;
        trc::derniere_erreur() = message;
    }
    return r;
}

extern "C" int trc_diffusion_jeton(trc_diffusion* m, trc_vue x, trc_vue residu, void* flux) {
    if (m == nullptr) return trc::usage("moteur nul");
    for (uint32_t l = 0; l < m->couches.size(); ++l) TRC_OK_OU_RENDRE(trc_diffusion_couche(m, l, x, residu, flux, nullptr));
    return TRC_OK;
}

extern "C" int trc_diffusion_stats(const trc_diffusion* m, trc_stats_diffusion* s) {
    if (m == nullptr || s == nullptr) return trc::usage("moteur ou sortie nuls");
    *s = m->st;
    return TRC_OK;
}

extern "C" int trc_diffusion_controle(const trc_diffusion* m, uint32_t* mots) {
    if (m == nullptr || mots == nullptr) return trc::usage("moteur ou sortie nuls");
    TRC_HIP(hipMemcpy(mots, m->controle, 16, hipMemcpyDeviceToHost));
    return TRC_OK;
}
