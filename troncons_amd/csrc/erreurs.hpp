// erreurs.hpp — status codes and the per-thread last-error message of the C-ABI
// (mirrors trc_cuda::Erreur: Usage before any call, HIP errors with the runtime's name and text).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/troncons_hip.h"

namespace trc {

std::string& derniere_erreur();
int& dernier_code_hip();  // hipError_t of the thread's last error, 0 when it was not a HIP error

inline int usage(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    derniere_erreur() = std::string("usage : ") + buf;
    dernier_code_hip() = 0;
    return TRC_ERREUR_USAGE;
}

inline int erreur_hip(const char* appel, hipError_t e) {
    char buf[512];
    snprintf(buf, sizeof(buf), "%s : %s (%d) : %s", appel, hipGetErrorName(e), int(e), hipGetErrorString(e));
    derniere_erreur() = buf;
    dernier_code_hip() = int(e);
    return e == hipErrorNoDevice || e == hipErrorInsufficientDriver ? TRC_ERREUR_PILOTE : TRC_ERREUR_HIP;
}

// Status of the last launch on this thread.
inline int apres_lancement(const char* nom) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return erreur_hip(nom, e);
    return TRC_OK;
}

#define TRC_VERIFIER(cond, ...)                 \
    do {                                        \
        if (!(cond)) return ::trc::usage(__VA_ARGS__); \
    } while (0)

}  // namespace trc
