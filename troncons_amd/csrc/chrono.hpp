// chrono.hpp — optional per-kernel timing of the fused entry points (see chrono.cpp).
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

namespace trc {
bool chrono_actif();
// Two events from the pool when timing is on (false when off).
bool chrono_paire(hipEvent_t* debut, hipEvent_t* fin);
// Files a recorded pair under `nom` (a string literal).
void chrono_classer(hipEvent_t debut, hipEvent_t fin, const char* nom);
}  // namespace trc

// Launches a kernel on stream f — through hipExtLaunchKernel with start/stop events when timing is
// on — and returns from the enclosing function on a launch error.
#define TRC_LANCER_N(nom, noyau, grille, bloc, f, ...)                                    \
    do {                                                                                  \
        hipEvent_t d_ = nullptr, e_ = nullptr;                                            \
        const bool c_ = ::trc::chrono_paire(&d_, &e_);                                    \
        if (c_)                                                                           \
            hipExtLaunchKernelGGL(noyau, grille, bloc, 0, f, d_, e_, 0, __VA_ARGS__);     \
        else                                                                              \
            hipLaunchKernelGGL(noyau, grille, bloc, 0, f, __VA_ARGS__);                   \
        const int r_ = ::trc::apres_lancement(#noyau);                                    \
        if (c_) ::trc::chrono_classer(d_, e_, nom);                                       \
        if (r_ != TRC_OK) return r_;                                                      \
    } while (0)
#define TRC_LANCER(noyau, grille, bloc, f, ...) TRC_LANCER_N(#noyau, noyau, grille, bloc, f, __VA_ARGS__)
