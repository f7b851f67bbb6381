// chrono.hpp — optional per-kernel event timing of the fused entry points (see chrono.cpp).
#pragma once

#include <hip/hip_runtime.h>

namespace trc {
bool chrono_actif();
// Records a start event on f if timing is on; returns a token (nullptr when off).
void* chrono_debut(hipStream_t f);
// Records the end event and files the pair under `nom` (a string literal).
void chrono_fin(void* jeton, const char* nom, hipStream_t f);
}  // namespace trc

// Launches a kernel on stream f, bracketed by chronogram events when timing is on, and returns
// from the enclosing function on a launch error.
#define TRC_LANCER_N(nom, noyau, grille, bloc, f, ...)                                    \
    do {                                                                                  \
        void* jeton_ = ::trc::chrono_debut(f);                                            \
        hipLaunchKernelGGL(noyau, grille, bloc, 0, f, __VA_ARGS__);                       \
        const int r_ = ::trc::apres_lancement(#noyau);                                    \
        ::trc::chrono_fin(jeton_, nom, f);                                                \
        if (r_ != TRC_OK) return r_;                                                      \
    } while (0)
#define TRC_LANCER(noyau, grille, bloc, f, ...) TRC_LANCER_N(#noyau, noyau, grille, bloc, f, __VA_ARGS__)
