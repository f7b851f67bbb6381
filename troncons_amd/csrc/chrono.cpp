// chrono.cpp — per-kernel GPU timing of the fused entry points, off by default. The role of the
// reference's chronogram (trc-ordo records GPU event timestamps around each copy and decode,
// moteur/crates/trc-ordo/src/lib.rs:205-222): when enabled, every kernel launched by a fused entry
// point goes through hipExtLaunchKernel with a start and a stop event, which the runtime records
// at the kernel's own start and end (the execution time a kernel trace reports, without the
// dispatch gaps around it); trc_chrono_recolter() waits for them and returns the summed
// milliseconds and launch count per kernel name.
#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "chrono.hpp"
#include "erreurs.hpp"

namespace trc {
namespace {

struct Mesure {
    const char* nom;
    hipEvent_t debut, fin;
};

struct Chrono {
    std::mutex m;
    bool actif = false;
    std::vector<hipEvent_t> libres;
    std::vector<Mesure> en_cours;
    std::map<std::string, std::pair<double, uint64_t>> totaux;
};

Chrono& chrono() {
    static Chrono c;
    return c;
}

hipEvent_t prendre(Chrono& c) {
    if (!c.libres.empty()) {
        hipEvent_t e = c.libres.back();
        c.libres.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

}  // namespace

bool chrono_actif() { return chrono().actif; }

bool chrono_paire(hipEvent_t* debut, hipEvent_t* fin) {
    Chrono& c = chrono();
    std::lock_guard<std::mutex> g(c.m);
    if (!c.actif) return false;
    *debut = prendre(c);
    *fin = prendre(c);
    if (*debut == nullptr || *fin == nullptr) {
        if (*debut) c.libres.push_back(*debut);
        if (*fin) c.libres.push_back(*fin);
        return false;
    }
    return true;
}

void chrono_classer(hipEvent_t debut, hipEvent_t fin, const char* nom) {
    Chrono& c = chrono();
    std::lock_guard<std::mutex> g(c.m);
    c.en_cours.push_back({nom, debut, fin});
}

}  // namespace trc

extern "C" void trc_chrono(int actif) {
    trc::Chrono& c = trc::chrono();
    std::lock_guard<std::mutex> g(c.m);
    c.actif = actif != 0;
}

// Waits for every recorded pair, adds it to the per-name totals, and copies at most `max` entries
// (name, total ms, launches) out; returns the number of names. noms: max x 64 chars.
extern "C" int trc_chrono_recolter(char* noms, double* ms, uint64_t* lancements, int max, int remettre_a_zero) {
    trc::Chrono& c = trc::chrono();
    std::lock_guard<std::mutex> g(c.m);
    for (auto& me : c.en_cours) {
        float t = 0.0f;
        if (hipEventSynchronize(me.fin) == hipSuccess && hipEventElapsedTime(&t, me.debut, me.fin) == hipSuccess) {
            auto& tot = c.totaux[me.nom];
            tot.first += t;
            tot.second += 1;
        }
        c.libres.push_back(me.debut);
        c.libres.push_back(me.fin);
    }
    c.en_cours.clear();
    int n = 0;
    for (auto& kv : c.totaux) {
        if (n >= max) break;
        if (noms) {
            std::strncpy(noms + 64 * n, kv.first.c_str(), 63);
            noms[64 * n + 63] = 0;
        }
        if (ms) ms[n] = kv.second.first;
        if (lancements) lancements[n] = kv.second.second;
        ++n;
    }
    if (remettre_a_zero) c.totaux.clear();
    return n;
}
