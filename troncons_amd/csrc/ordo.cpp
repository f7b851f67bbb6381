// ordo.cpp — the streaming scheduler of the expert path (host C++ over HIP): a token through the
// MoE part of every layer of a .trc file, with the experts streamed from the file and kept decoded
// in a slot cache in HBM.
//
// Role of the reference's Moteur::pas (moteur/crates/trc-ordo/src/lib.rs:1054-1280) for the expert
// path, per layer:
//   1. router on the compute stream (gemv_f32 + routeur_topk), whose kernel writes the k indices and
//      a sequence word into a mapped host mailbox; the host waits for the router's event and reads
//      the mailbox (the one device -> host wait per layer, lib.rs:1108-1128);
//   2. the cache decides per expert (lib.rs:1139): VRAM hit, RAM hit (coded part already in a
//      pinned warm entry) or disk miss;
//   3. the disk misses are read at once by reader threads (pread on the shared file descriptor) into
//      their warm entries, or into per-place pinned arrival buffers without a RAM stage
//      (lib.rs:1164-1187); each part, once on the host, is copied on the copy stream into a device
//      arrival buffer and decoded into its slot on the compute stream after that copy's event
//      (envoyer_et_decoder, lib.rs:1328-1368);
//   4. pret for every miss, then the layer's expert MLPs over the decoded slots — the reference's
//      fin_couche (trc-modele/src/lib.rs:533-553): gemv gate and up for all k experts in one batched
//      launch, swiglu_oai, gemv down batched, then the ordered combine into the residual — and
//      liberer (lib.rs:1261-1267).
// Buffer reuse needs no extra waits: everything of layer l on the compute stream precedes the
// router of layer l + 1, whose mailbox the host waits for before reusing any buffer of layer l.
#include <hip/hip_runtime.h>

#include <cmath>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <condition_variable>
#include <cstring>
#include <deque>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "commun.hpp"
#include "erreurs.hpp"

namespace {

using horloge = std::chrono::steady_clock;

double us_depuis(horloge::time_point t0) {
    return std::chrono::duration<double, std::micro>(horloge::now() - t0).count();
}

#define TRC_HIP(appel)                                              \
    do {                                                            \
        const hipError_t e_ = (appel);                              \
        if (e_ != hipSuccess) return ::trc::erreur_hip(#appel, e_); \
    } while (0)

#define TRC_OK_OU_RENDRE(expr)     \
    do {                           \
        const int r_ = (expr);     \
        if (r_ != TRC_OK) return r_; \
    } while (0)

// A pool of reader threads: parts are read with pread (thread-safe on the shared descriptor).
class Lecteurs {
public:
    struct Requete {
        uint16_t couche, expert;
        uint8_t* dst;
        uint64_t cap;
        int verifier;
        uint32_t n;  // index of the miss in the layer
    };
    struct Fin {
        uint32_t n;
        int statut;
        uint64_t octets;
        std::string message;
    };

    Lecteurs(const trc_fichier* f, unsigned n) : f_(f) {
        for (unsigned i = 0; i < n; ++i) fils_.emplace_back([this] { boucle(); });
    }
    ~Lecteurs() {
        {
            std::lock_guard<std::mutex> g(m_);
            fin_ = true;
        }
        cv_.notify_all();
        for (auto& t : fils_) t.join();
    }
    // soumettre / attendre / vider are called by the engine's thread only.
    void soumettre(const Requete& r) {
        {
            std::lock_guard<std::mutex> g(m_);
            file_.push_back(r);
        }
        ++en_cours_;
        cv_.notify_one();
    }
    Fin attendre() {
        std::unique_lock<std::mutex> g(m_);
        cv_fini_.wait(g, [this] { return !finis_.empty(); });
        Fin x = std::move(finis_.front());
        finis_.pop_front();
        --en_cours_;
        return x;
    }
    // Waits for every submitted read that has not been taken by attendre(): after an error, no
    // reader thread writes into the engine's buffers any more.
    void vider() {
        while (en_cours_ > 0) attendre();
    }

private:
    void boucle() {
        for (;;) {
            Requete r;
            {
                std::unique_lock<std::mutex> g(m_);
                cv_.wait(g, [this] { return fin_ || !file_.empty(); });
                if (fin_ && file_.empty()) return;
                r = file_.front();
                file_.pop_front();
            }
            Fin x{r.n, TRC_OK, 0, {}};
            x.statut = trc_fichier_lire_partie(f_, r.couche, r.expert, 1, r.dst, r.cap, r.verifier, &x.octets);
            if (x.statut != TRC_OK) x.message = trc_derniere_erreur();
            {
                std::lock_guard<std::mutex> g(m_);
                finis_.push_back(std::move(x));
            }
            cv_fini_.notify_one();
        }
    }
    const trc_fichier* f_;
    std::vector<std::thread> fils_;
    std::mutex m_;
    std::condition_variable cv_, cv_fini_;
    std::deque<Requete> file_;
    std::deque<Fin> finis_;
    bool fin_ = false;
    uint64_t en_cours_ = 0;
};

}  // namespace

struct trc_ordo {
    const trc_fichier* f = nullptr;
    trc_config_ordo cfg{};
    trc_dims_expert dims{};
    uint32_t L = 0, E = 0, k = 0, R = 0, C = 0, D = 0;
    uint64_t te = 0, lg_max = 0;
    trc_disposition disp[3];
    trc_cache* cache = nullptr;
    std::unique_ptr<Lecteurs> lecteurs;
    bool en_echec = false;       // an error stopped a token: every later token is refused
    std::string message_echec;
    hipStream_t copie = nullptr;
    hipEvent_t ev_routeur = nullptr;
    std::vector<hipEvent_t> ev_copie;
    // device
    uint8_t* emplacements = nullptr;
    std::vector<uint8_t*> arrivees;
    uint32_t* luts = nullptr;     // L x u32[3][4][4096]
    float* routeurs = nullptr;    // L x E x C
    float* logits = nullptr;
    uint32_t* idx = nullptr;
    float* poids = nullptr;
    float *g = nullptr, *u = nullptr, *a = nullptr, *sorties = nullptr;
    trc_desc_gemv* descs = nullptr;
    uint32_t* controle = nullptr;
    // pinned host
    uint8_t* tiedes = nullptr;         // cfg.tiedes entries of lg_max bytes
    uint8_t* arrivees_hote = nullptr;  // k entries of lg_max bytes (disk misses without a warm entry)
    uint32_t* boite = nullptr;         // mapped mailbox: [0] sequence, [1..k] indices, [k+1..2k] weights
    uint32_t* boite_carte = nullptr;
    trc_desc_gemv* descs_hote = nullptr;
    uint32_t sequence = 0;
    uint64_t jeton = 0;
    trc_stats_ordo st{};
    std::vector<uint16_t> trace;
    // prefetch (cfg.prechargement): two sets of k pinned buffers, set l % 2 for layer l's parts
    struct Prechargement {
        int32_t couche = -1;  // -1: empty
        uint16_t expert = 0;
        bool en_vol = false;       // its read has not landed
        bool pris = false;         // a miss of its layer took it
        int32_t attendu_par = -1;  // the miss waiting for its read to land
        int statut = TRC_OK;
        uint64_t octets = 0;
        std::string message;
    };
    static constexpr uint32_t PF_JETON = 1u << 16;     // reader requests from here on are prefetches
    static constexpr uint32_t BOITE_PREDICTION = 64;  // the prediction's mailbox, 256 bytes in
    static constexpr float EPS_PREDICTION = 1e-5f;    // gpt-oss's RMSNorm epsilon
    std::vector<Prechargement> pf;
    uint8_t* pf_hote = nullptr;
    float* normes = nullptr;  // L x D post-attention norm weights
    float *h2p = nullptr, *logits_p = nullptr, *poids_p = nullptr;
    uint32_t* idx_p = nullptr;
    // cache-biased router (cfg.avec_biais_cache): beta per expert of the layer, pinned then device
    float* biais_hote = nullptr;
    float* biais_carte = nullptr;

    ~trc_ordo() {
        lecteurs.reset();
        if (cache) trc_cache_detruire(cache);
        (void)hipDeviceSynchronize();
        for (hipEvent_t e : ev_copie) (void)hipEventDestroy(e);
        if (ev_routeur) (void)hipEventDestroy(ev_routeur);
        if (copie) (void)hipStreamDestroy(copie);
        void* dev[] = {emplacements, luts, routeurs, logits, idx, poids, g, u, a, sorties, descs, controle,
                       normes, h2p, logits_p, poids_p, idx_p, biais_carte};
        for (void* p : dev)
            if (p) (void)hipFree(p);
        for (uint8_t* p : arrivees)
            if (p) (void)hipFree(p);
        void* hote[] = {tiedes, arrivees_hote, boite, descs_hote, pf_hote, biais_hote};
        for (void* p : hote)
            if (p) (void)hipHostFree(p);
    }

    uint8_t* emplacement(uint32_t s) const { return emplacements + uint64_t(s) * te; }

    int allouer() {
        const uint32_t K = k;
        TRC_HIP(hipStreamCreateWithFlags(&copie, hipStreamNonBlocking));
        TRC_HIP(hipEventCreateWithFlags(&ev_routeur, hipEventDisableTiming));
        ev_copie.assign(K, nullptr);
        for (uint32_t i = 0; i < K; ++i) TRC_HIP(hipEventCreateWithFlags(&ev_copie[i], hipEventDisableTiming));
        TRC_HIP(hipMalloc(&emplacements, uint64_t(cfg.emplacements) * te));
        arrivees.assign(K, nullptr);
        for (uint32_t i = 0; i < K; ++i) TRC_HIP(hipMalloc(&arrivees[i], lg_max));
        TRC_HIP(hipMalloc(&luts, uint64_t(L) * trc::LUTS_PAR_COUCHE * 4));
        TRC_HIP(hipMalloc(&routeurs, uint64_t(L) * E * C * 4));
        TRC_HIP(hipMalloc(&logits, 4ull * E));
        TRC_HIP(hipMalloc(&idx, 64));
        TRC_HIP(hipMalloc(&poids, 64));
        TRC_HIP(hipMalloc(&g, 4ull * K * R));
        TRC_HIP(hipMalloc(&u, 4ull * K * R));
        TRC_HIP(hipMalloc(&a, 4ull * K * R));
        TRC_HIP(hipMalloc(&sorties, 4ull * K * D));
        TRC_HIP(hipMalloc(&descs, sizeof(trc_desc_gemv) * 3 * K));
        TRC_HIP(hipMalloc(&controle, 16));
        TRC_HIP(hipMemset(controle, 0, 16));
        if (cfg.tiedes) TRC_HIP(hipHostMalloc(&tiedes, uint64_t(cfg.tiedes) * lg_max, hipHostMallocDefault));
        TRC_HIP(hipHostMalloc(&arrivees_hote, uint64_t(K) * lg_max, hipHostMallocDefault));
        TRC_HIP(hipHostMalloc(&boite, 4096, hipHostMallocMapped | hipHostMallocCoherent));
        std::memset(boite, 0, 4096);
        TRC_HIP(hipHostGetDevicePointer(reinterpret_cast<void**>(&boite_carte), boite, 0));
        TRC_HIP(hipHostMalloc(&descs_hote, sizeof(trc_desc_gemv) * 3 * K, hipHostMallocDefault));
        // per layer: LUTs from TABLES, router from RÉSIDENTS (bf16 rows widened to f32)
        std::vector<uint16_t> fr(3 * 4 * 256);
        std::vector<uint32_t> lh(trc::LUTS_PAR_COUCHE);
        std::vector<float> rf(uint64_t(E) * C);
        const trc_resident* res = trc_fichier_residents(f);
        const uint32_t n_res = trc_fichier_n_residents(f);
        for (uint32_t l = 0; l < L; ++l) {
            TRC_OK_OU_RENDRE(trc_fichier_freqs_couche(f, uint16_t(l), fr.data()));
            const uint16_t* pf[12];
            for (int i = 0; i < 12; ++i) pf[i] = fr.data() + 256 * i;
            TRC_OK_OU_RENDRE(trc_luts_couche(pf, lh.data()));
            TRC_HIP(hipMemcpy(luts + uint64_t(l) * trc::LUTS_PAR_COUCHE, lh.data(), lh.size() * 4, hipMemcpyHostToDevice));
            char nom[64];
            snprintf(nom, sizeof(nom), "blk.%u.ffn_gate_inp.weight", l);
            const trc_resident* r = nullptr;
            for (uint32_t i = 0; i < n_res; ++i)
                if (strncmp(res[i].nom, nom, 64) == 0) r = &res[i];
            if (r == nullptr) return trc::usage("routeur %s absent des residents", nom);
            if (r->type_ggml != 30 || r->ne[0] != C || r->ne[1] != E || r->octets != 2ull * E * C)
                return trc::usage("routeur %s : bf16 %u x %u attendu", nom, E, C);
            std::vector<uint16_t> b(uint64_t(E) * C);
            TRC_OK_OU_RENDRE(trc_fichier_lire(f, trc_fichier_debut_donnees(f) + r->decalage, r->octets, b.data()));
            for (uint64_t i = 0; i < b.size(); ++i) {
                const uint32_t bits = uint32_t(b[i]) << 16;
                std::memcpy(&rf[i], &bits, 4);
            }
            TRC_HIP(hipMemcpy(routeurs + uint64_t(l) * E * C, rf.data(), rf.size() * 4, hipMemcpyHostToDevice));
        }
        if (cfg.avec_biais_cache) {
            TRC_HIP(hipHostMalloc(&biais_hote, 4ull * E, hipHostMallocDefault));
            TRC_HIP(hipMalloc(&biais_carte, 4ull * E));
        }
        if (cfg.prechargement) {
            pf.assign(2 * K, Prechargement{});
            TRC_HIP(hipHostMalloc(&pf_hote, uint64_t(2 * K) * lg_max, hipHostMallocDefault));
            TRC_HIP(hipMalloc(&normes, uint64_t(L) * D * 4));
            TRC_HIP(hipMalloc(&h2p, 4ull * D));
            TRC_HIP(hipMalloc(&logits_p, 4ull * E));
            TRC_HIP(hipMalloc(&idx_p, 64));
            TRC_HIP(hipMalloc(&poids_p, 64));
            // the post-attention norms from RÉSIDENTS (f32[D]) when the file holds them, else 1
            std::vector<float> w(D);
            for (uint32_t l = 0; l < L; ++l) {
                char nom[64];
                snprintf(nom, sizeof(nom), "blk.%u.post_attention_norm.weight", l);
                const trc_resident* r = nullptr;
                for (uint32_t i = 0; i < n_res; ++i)
                    if (strncmp(res[i].nom, nom, 64) == 0) r = &res[i];
                if (r == nullptr) {
                    std::fill(w.begin(), w.end(), 1.0f);
                } else {
                    if (r->type_ggml != 0 || r->ne[0] != D || r->octets != 4ull * D)
                        return trc::usage("norme %s : f32 de %u attendu", nom, D);
                    TRC_OK_OU_RENDRE(trc_fichier_lire(f, trc_fichier_debut_donnees(f) + r->decalage, r->octets, w.data()));
                }
                TRC_HIP(hipMemcpy(normes + uint64_t(l) * D, w.data(), 4ull * D, hipMemcpyHostToDevice));
            }
        }
        return TRC_OK;
    }

    // envoyer_et_decoder: the part is on the host at `src`; copy it to arrival i, decode it into s.
    int envoyer_et_decoder(uint32_t l, uint32_t i, const uint8_t* src, uint64_t octets, uint32_t s, void* flux) {
        uint32_t g1[3], g2[3];
        TRC_OK_OU_RENDRE(trc_grilles_depuis_partie(src, octets, g1, g2));
        TRC_HIP(hipMemcpyAsync(arrivees[i], src, octets, hipMemcpyHostToDevice, copie));
        TRC_HIP(hipEventRecord(ev_copie[i], copie));
        const hipStream_t f = reinterpret_cast<hipStream_t>(flux);
        TRC_HIP(hipStreamWaitEvent(f, ev_copie[i], 0));
        const trc_vue vp{uint64_t(reinterpret_cast<uintptr_t>(arrivees[i])), octets};
        const trc_vue ve{uint64_t(reinterpret_cast<uintptr_t>(emplacement(s))), te};
        const trc_vue vl{uint64_t(reinterpret_cast<uintptr_t>(luts + uint64_t(l) * trc::LUTS_PAR_COUCHE)),
                         uint64_t(trc::LUTS_PAR_COUCHE) * 4};
        const trc_vue vc{uint64_t(reinterpret_cast<uintptr_t>(controle)), 16};
        TRC_OK_OU_RENDRE(trc_decoder_expert_grilles(vp, ve, vl, &dims, vc, g1, g2, flux));
        st.octets_copies += octets;
        st.decodages += 1;
        return TRC_OK;
    }

    int couche(uint32_t l, const trc_vue& x, const trc_vue& residu, void* flux) {
        const hipStream_t fl = reinterpret_cast<hipStream_t>(flux);
        auto vue = [](const void* p, uint64_t n) { return trc_vue{uint64_t(reinterpret_cast<uintptr_t>(p)), n}; };
        const auto t_emis = horloge::now();
        // 1. router, mailbox
        sequence = sequence + 1 == 0 ? 1 : sequence + 1;
        const uint32_t seq = sequence;
        TRC_OK_OU_RENDRE(trc_gemv_f32(vue(routeurs + uint64_t(l) * E * C, 4ull * E * C), x, trc_vue{0, 0},
                                      vue(logits, 4ull * E), E, C, flux));
        if (cfg.avec_biais_cache) {
            // beta on each of layer l's experts in a VRAM slot just before its request (the cache
            // after layer l-1 of this token: causal), sent before the router (lib.rs:1089-1100); the
            // pinned vector is free again: its previous copy precedes the router event waited for
            for (uint32_t e = 0; e < E; ++e)
                biais_hote[e] = trc_cache_emplacement_de(cache, uint16_t(l), uint16_t(e)) >= 0 ? cfg.biais_cache : 0.0f;
            TRC_HIP(hipMemcpyAsync(biais_carte, biais_hote, 4ull * E, hipMemcpyHostToDevice, fl));
            TRC_OK_OU_RENDRE(trc_routeur_topk_biais(vue(logits, 4ull * E), vue(biais_carte, 4ull * E), E, k, vue(idx, 64),
                                                    vue(poids, 64), uint64_t(reinterpret_cast<uintptr_t>(boite_carte)),
                                                    seq, flux));
        } else {
            TRC_OK_OU_RENDRE(trc_routeur_topk(vue(logits, 4ull * E), E, k, vue(idx, 64), vue(poids, 64),
                                              uint64_t(reinterpret_cast<uintptr_t>(boite_carte)), seq, flux));
        }
        // Modele::predire (trc-modele/src/lib.rs:570-579): layer l+1's router over the residual
        // normed with l+1's post-attention norm, into the second mailbox; x and the residual untouched
        const bool predire = cfg.prechargement && l + 1 < L;
        if (predire) {
            TRC_OK_OU_RENDRE(trc_rmsnorm(residu, vue(normes + uint64_t(l + 1) * D, 4ull * D), vue(h2p, 4ull * D), D, 1,
                                         EPS_PREDICTION, flux));
            TRC_OK_OU_RENDRE(trc_gemv_f32(vue(routeurs + uint64_t(l + 1) * E * C, 4ull * E * C), vue(h2p, 4ull * C),
                                          trc_vue{0, 0}, vue(logits_p, 4ull * E), E, C, flux));
            TRC_OK_OU_RENDRE(trc_routeur_topk(vue(logits_p, 4ull * E), E, k, vue(idx_p, 64), vue(poids_p, 64),
                                              uint64_t(reinterpret_cast<uintptr_t>(boite_carte + BOITE_PREDICTION)),
                                              seq, flux));
        }
        TRC_HIP(hipEventRecord(ev_routeur, fl));
        st.us_emission += us_depuis(t_emis);
        const auto t0 = horloge::now();
        TRC_HIP(hipEventSynchronize(ev_routeur));
        const volatile uint32_t* bv = boite;
        if (bv[0] != seq) return trc::usage("couche %u : boite a la sequence %u, %u attendue", l, bv[0], seq);
        uint16_t experts[8];
        for (uint32_t i = 0; i < k; ++i) {
            const uint32_t e = bv[1 + i];
            if (e >= E) return trc::usage("couche %u : expert %u hors de [0, %u)", l, e, E);
            experts[i] = uint16_t(e);
        }
        uint16_t predits[8] = {};
        if (predire) {
            if (bv[BOITE_PREDICTION] != seq)
                return trc::usage("couche %u : boite de prediction a la sequence %u, %u attendue", l, bv[BOITE_PREDICTION],
                                  seq);
            for (uint32_t i = 0; i < k; ++i) predits[i] = uint16_t(bv[BOITE_PREDICTION + 1 + i]);
        }
        st.us_attente_routeur += us_depuis(t0);
        trace.insert(trace.end(), experts, experts + k);
        // 2. decisions
        trc_decision d[8];
        TRC_OK_OU_RENDRE(trc_cache_demander(cache, uint16_t(l), experts, k, jeton * L + l, d));
        // 3. misses: disk reads submitted at once; RAM hits sent at once; disk misses sent as they land.
        // With prefetch, a disk miss without a warm entry whose part was read ahead (set l % 2) takes
        // it from the prefetch buffer: at once if the read has landed, else when it lands.
        const auto t_es = horloge::now();
        int32_t pf_de[8];
        for (uint32_t i = 0; i < k; ++i) {
            pf_de[i] = -1;
            if (!cfg.prechargement || d[i].sorte != TRC_DECISION_DEFAUT_DISQUE || d[i].tiede >= 0) continue;
            for (uint32_t s = (l % 2u) * k; s < (l % 2u + 1u) * k; ++s)
                if (pf[s].couche == int32_t(l) && pf[s].expert == experts[i] && !pf[s].pris) {
                    pf_de[i] = int32_t(s);
                    pf[s].pris = true;
                    st.pf_utiles += 1;
                    break;
                }
        }
        uint32_t en_vol = 0;  // completions this layer waits for: its own reads and the prefetches it took
        for (uint32_t i = 0; i < k; ++i) {
            if (d[i].sorte != TRC_DECISION_DEFAUT_DISQUE || pf_de[i] >= 0) continue;
            uint8_t* dst = d[i].tiede >= 0 ? tiedes + uint64_t(d[i].tiede) * lg_max : arrivees_hote + uint64_t(i) * lg_max;
            lecteurs->soumettre({uint16_t(l), experts[i], dst, lg_max, cfg.verifier, i});
            ++en_vol;
        }
        // From here on an error is kept in `echec` (the first one wins) and returned only once every
        // read this layer submitted or took over has landed, so that no completion is left for a later
        // token to pick up with this layer's indices.
        int echec = TRC_OK;
        std::string message;
        auto noter_echec = [&](int r, const std::string& m) {
            if (r != TRC_OK && echec == TRC_OK) {
                echec = r;
                message = m;
            }
        };
        for (uint32_t i = 0; i < k && echec == TRC_OK; ++i) {
            if (d[i].sorte != TRC_DECISION_DEFAUT_RAM) continue;
            const trc_entree_repertoire* en = trc_fichier_entree(f, uint16_t(l), experts[i]);
            const int r = envoyer_et_decoder(l, i, tiedes + uint64_t(d[i].tiede) * lg_max, en->longueur[0],
                                             d[i].emplacement, flux);
            if (r != TRC_OK) noter_echec(r, trc_derniere_erreur());
        }
        for (uint32_t i = 0; i < k; ++i) {
            if (pf_de[i] < 0) continue;
            Prechargement& p = pf[pf_de[i]];
            if (p.en_vol) {
                p.attendu_par = int32_t(i);
                ++en_vol;
                continue;
            }
            if (echec != TRC_OK) continue;
            if (p.statut != TRC_OK) {
                noter_echec(p.statut, p.message);
                continue;
            }
            const int r = envoyer_et_decoder(l, i, pf_hote + uint64_t(pf_de[i]) * lg_max, p.octets,
                                             d[i].emplacement, flux);
            if (r != TRC_OK) noter_echec(r, trc_derniere_erreur());
        }
        auto traiter = [&](Lecteurs::Fin x) {
            const uint8_t* src;
            uint32_t i;
            if (x.n >= PF_JETON) {
                Prechargement& p = pf[x.n - PF_JETON];
                p.en_vol = false;
                p.statut = x.statut;
                p.octets = x.octets;
                if (x.statut != TRC_OK) p.message = x.message;
                if (p.attendu_par < 0) return;  // a read ahead nobody waits for (yet)
                i = uint32_t(p.attendu_par);
                p.attendu_par = -1;
                src = pf_hote + uint64_t(x.n - PF_JETON) * lg_max;
            } else {
                i = x.n;
                if (x.statut == TRC_OK) {
                    st.octets_lus += x.octets;
                    st.lectures += 1;
                }
                src = d[i].tiede >= 0 ? tiedes + uint64_t(d[i].tiede) * lg_max : arrivees_hote + uint64_t(i) * lg_max;
            }
            --en_vol;
            if (x.statut != TRC_OK) {
                noter_echec(x.statut, x.message);
                return;
            }
            if (echec != TRC_OK) return;
            const int r = envoyer_et_decoder(l, i, src, x.octets, d[i].emplacement, flux);
            if (r != TRC_OK) noter_echec(r, trc_derniere_erreur());
        };
        // the reads ahead for layer l+1, queued behind layer l's own (Moteur::pas, lib.rs:1194-1215):
        // set (l+1) % 2 is reused once the reads still landing in it have landed; its copies to the
        // device (layer l-1) are over, since the router event waited for above follows the decodes
        // that waited for them
        if (predire) {
            const uint32_t ens = (l + 1u) % 2u;
            auto ensemble_en_vol = [&] {
                for (uint32_t s = ens * k; s < (ens + 1u) * k; ++s)
                    if (pf[s].en_vol) return true;
                return false;
            };
            while (ensemble_en_vol()) traiter(lecteurs->attendre());
            for (uint32_t i = 0; i < k; ++i) {
                const uint32_t s = ens * k + i;
                pf[s] = Prechargement{};
                const uint16_t e = predits[i];
                if (e >= E || trc_cache_emplacement_de(cache, uint16_t(l + 1), e) >= 0 ||
                    trc_cache_tiede_de(cache, uint16_t(l + 1), e) >= 0)
                    continue;
                lecteurs->soumettre({uint16_t(l + 1), e, pf_hote + uint64_t(s) * lg_max, lg_max, cfg.verifier, PF_JETON + s});
                pf[s].couche = int32_t(l + 1);
                pf[s].expert = e;
                pf[s].en_vol = true;
                const uint64_t lg = trc_fichier_entree(f, uint16_t(l + 1), e)->longueur[0];
                st.pf_emis += 1;
                st.pf_octets += lg;
                st.lectures += 1;
                st.octets_lus += lg;
            }
        }
        while (en_vol > 0) traiter(lecteurs->attendre());
        if (echec != TRC_OK) {
            trc::derniere_erreur() = message;
            return echec;
        }
        st.us_lectures += us_depuis(t_es);
        const auto t_fin = horloge::now();
        for (uint32_t i = 0; i < k; ++i)
            if (d[i].sorte != TRC_DECISION_SUCCES) TRC_OK_OU_RENDRE(trc_cache_pret(cache, d[i].emplacement));
        // 4. fin_couche over the decoded slots
        for (uint32_t i = 0; i < k; ++i) {
            const uint8_t* s = emplacement(d[i].emplacement);
            descs_hote[2 * i] = {uint64_t(reinterpret_cast<uintptr_t>(s + disp[0].base)), x.adresse,
                                 uint64_t(reinterpret_cast<uintptr_t>(g + uint64_t(i) * R)), R, C};
            descs_hote[2 * i + 1] = {uint64_t(reinterpret_cast<uintptr_t>(s + disp[1].base)), x.adresse,
                                     uint64_t(reinterpret_cast<uintptr_t>(u + uint64_t(i) * R)), R, C};
            descs_hote[2 * k + i] = {uint64_t(reinterpret_cast<uintptr_t>(s + disp[2].base)),
                                     uint64_t(reinterpret_cast<uintptr_t>(a + uint64_t(i) * R)),
                                     uint64_t(reinterpret_cast<uintptr_t>(sorties + uint64_t(i) * D)), D, R};
        }
        TRC_HIP(hipMemcpyAsync(descs, descs_hote, sizeof(trc_desc_gemv) * 3 * k, hipMemcpyHostToDevice, fl));
        TRC_OK_OU_RENDRE(trc_gemv_lot(vue(descs, sizeof(trc_desc_gemv) * 2 * k), 2 * k, R, flux));
        TRC_OK_OU_RENDRE(trc_swiglu_oai(vue(g, 4ull * k * R), vue(u, 4ull * k * R), vue(a, 4ull * k * R), k * R, flux));
        TRC_OK_OU_RENDRE(trc_gemv_lot(vue(descs + 2 * k, sizeof(trc_desc_gemv) * k), k, D, flux));
        TRC_OK_OU_RENDRE(trc_combiner(residu, vue(sorties, 4ull * k * D), D, vue(poids, 4ull * k), k, D, flux));
        trc_cache_liberer_couche(cache, uint16_t(l));
        st.us_emission += us_depuis(t_fin);
        return TRC_OK;
    }
};

extern "C" {

int trc_ordo_creer(const trc_fichier* f, const trc_config_ordo* cfg, trc_ordo** sortie) {
    if (f == nullptr || cfg == nullptr || sortie == nullptr) return trc::usage("pointeur nul");
    *sortie = nullptr;
    const trc_entete_fichier* e = trc_fichier_entete(f);
    if (e->matrices != 3 || e->niveaux != 1 || (e->drapeaux & (TRC_DRAPEAU_BRUT | TRC_DRAPEAU_RAPIDE)))
        return trc::usage("l'ordonnanceur lit un fichier code a un niveau, 3 matrices, ni brut ni rapide");
    auto o = std::make_unique<trc_ordo>();
    o->f = f;
    o->cfg = *cfg;
    for (int j = 0; j < 3; ++j) {
        o->dims.lignes[j] = e->lignes[j];
        o->dims.colonnes[j] = e->colonnes[j];
    }
    TRC_OK_OU_RENDRE(trc_dims_verifier(&o->dims));
    o->L = e->couches;
    o->E = e->experts;
    o->k = e->k;
    o->R = o->dims.lignes[0];
    o->C = o->dims.colonnes[0];
    o->D = o->dims.lignes[2];
    if (o->dims.lignes[1] != o->R || o->dims.colonnes[1] != o->C || o->dims.colonnes[2] != o->R)
        return trc::usage("formes : gate et up R x C, down D x R attendues");
    if (o->C % 4 != 0 || o->R % 4 != 0) return trc::usage("colonnes et lignes multiples de 4");
    if (o->k > 8 || o->E > 256) return trc::usage("top-%u sur %u experts (au plus 8 sur 256)", o->k, o->E);
    if (cfg->avec_biais_cache && !std::isfinite(cfg->biais_cache))
        return trc::usage("biais de cache : beta = %g n'est pas un nombre fini", double(cfg->biais_cache));
    if (cfg->avec_biais_cache && cfg->prechargement)
        return trc::usage("biais de cache et prechargement ne se combinent pas : la prediction est faite sans biais");
    if (cfg->prechargement && o->C != o->D)
        return trc::usage("prechargement : le residu (%u) doit avoir la largeur de l'entree du routeur (%u)", o->D, o->C);
    if (cfg->emplacements < o->k)
        return trc::usage("%u emplacements pour %u experts epingles par couche", cfg->emplacements, o->k);
    if (cfg->politique != TRC_POLITIQUE_LRU && cfg->politique != TRC_POLITIQUE_FIFO)
        return trc::usage("politique %d : LRU ou FIFO (Belady lit l'avenir)", cfg->politique);
    o->te = trc::al256(trc_taille_emplacement(&o->dims));
    for (int j = 0; j < 3; ++j) o->disp[j] = trc_disposition_j(&o->dims, uint32_t(j));
    const trc_entree_repertoire* rep = trc_fichier_repertoire(f);
    std::vector<uint64_t> tailles(uint64_t(o->L) * o->E);
    for (uint64_t i = 0; i < tailles.size(); ++i) {
        tailles[i] = rep[i].longueur[0];
        o->lg_max = std::max<uint64_t>(o->lg_max, rep[i].longueur[0]);
    }
    TRC_OK_OU_RENDRE(trc_cache_creer(cfg->emplacements, cfg->tiedes, cfg->politique, cfg->politique, nullptr, &o->cache));
    TRC_OK_OU_RENDRE(trc_cache_fixer_tailles(o->cache, uint16_t(o->L), uint16_t(o->E), tailles.data()));
    TRC_OK_OU_RENDRE(o->allouer());
    o->lecteurs = std::make_unique<Lecteurs>(f, std::max(1u, std::min(cfg->lecteurs ? cfg->lecteurs : o->k, 16u)));
    *sortie = o.release();
    return TRC_OK;
}

int trc_ordo_jeton(trc_ordo* o, trc_vue x, trc_vue residu, void* flux) {
    if (o == nullptr) return trc::usage("ordonnanceur nul");
    TRC_VERIFIER(x.adresse != 0 && x.adresse % 16 == 0 && x.octets >= 4ull * o->C, "x : %u f32 alignes sur 16", o->C);
    TRC_VERIFIER(residu.adresse != 0 && residu.octets >= 4ull * o->D, "residu : %u f32", o->D);
    if (o->en_echec) return trc::usage("ordonnanceur arrete par une erreur precedente : %s", o->message_echec.c_str());
    for (uint32_t l = 0; l < o->L; ++l) {
        const int r = o->couche(l, x, residu, flux);
        if (r != TRC_OK) {
            // fail-stop (the reference engine panics): the layer's reads still in flight are drained
            // so that no reader writes into the buffers later, and the engine refuses every later
            // token, since its cache holds slots that were never made ready
            const std::string m = trc_derniere_erreur();
            o->lecteurs->vider();
            (void)hipStreamSynchronize(o->copie);
            o->en_echec = true;
            o->message_echec = m;
            trc::derniere_erreur() = m;
            return r;
        }
    }
    o->jeton += 1;
    o->st.jetons += 1;
    return TRC_OK;
}

int trc_ordo_controle(trc_ordo* o, uint32_t mots[4], void* flux) {
    TRC_HIP(hipStreamSynchronize(reinterpret_cast<hipStream_t>(flux)));
    TRC_HIP(hipMemcpy(mots, o->controle, 16, hipMemcpyDeviceToHost));
    return TRC_OK;
}

trc_compteurs_cache trc_ordo_compteurs(const trc_ordo* o) { return trc_cache_compteurs(o->cache); }

trc_stats_ordo trc_ordo_stats(const trc_ordo* o) { return o->st; }

uint64_t trc_ordo_trace(const trc_ordo* o, uint16_t* choix, uint64_t max) {
    const uint64_t n = o->trace.size();
    if (choix) std::memcpy(choix, o->trace.data(), 2 * std::min(n, max));
    return n;
}

int trc_ordo_emplacement(const trc_ordo* o, uint16_t couche, uint16_t expert, trc_vue* vue) {
    const int64_t s = trc_cache_emplacement_de(o->cache, couche, expert);
    if (s < 0) return trc::usage("(%u, %u) absent de la VRAM", couche, expert);
    if (trc_cache_etat(o->cache, uint32_t(s)) != TRC_CACHE_PRESENT) return trc::usage("(%u, %u) en vol", couche, expert);
    vue->adresse = uint64_t(reinterpret_cast<uintptr_t>(o->emplacement(uint32_t(s))));
    vue->octets = o->te;
    return TRC_OK;
}

// The witness (mode témoin, trc-ordo/src/lib.rs:238-262, 1281-1300): the slot of a present expert
// copied to the host and fingerprinted, to compare with the directory entry.
int trc_ordo_temoin(const trc_ordo* o, uint16_t couche, uint16_t expert, void* flux, uint64_t* empreinte) {
    trc_vue v;
    TRC_OK_OU_RENDRE(trc_ordo_emplacement(o, couche, expert, &v));
    TRC_HIP(hipStreamSynchronize(reinterpret_cast<hipStream_t>(flux)));
    std::vector<uint8_t> h(v.octets);
    TRC_HIP(hipMemcpy(h.data(), reinterpret_cast<const void*>(uintptr_t(v.adresse)), v.octets, hipMemcpyDeviceToHost));
    *empreinte = trc_empreinte_emplacement(h.data(), &o->dims);
    return TRC_OK;
}

void trc_ordo_detruire(trc_ordo* o) { delete o; }

}  // extern "C"
