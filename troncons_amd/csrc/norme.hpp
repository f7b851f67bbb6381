// norme.hpp — the RMSNorm of one row by one block of 256 threads, with the reference's fixed
// reduction tree (passe.cuh:235-259): shared by the rmsnorm kernels and the launches that fold the
// norm into their prologue (the Q/K/V projections, the MoE router), so that all give its bits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace trc {

constexpr uint32_t FILS_NORME = 256;  // the block size these functions assume

// Sum of the block's 256 f64 values by the fixed tree (level k: value t += value t + k for t < k,
// k = 128 .. 1): levels 128 and 64 in LDS, levels 32 .. 1 as shuffles in wave 0 (lane t adds lane
// t + k, the same association). Every thread gets the sum.
__device__ __forceinline__ double somme_arbre_f64(double* part, double* total, double v) {
    const uint32_t t = threadIdx.x;
    part[t] = v;
    __syncthreads();
    if (t < 64u) {
        double u = (part[t] + part[t + 128u]) + (part[t + 64u] + part[t + 192u]);
#pragma unroll
        for (uint32_t k = 32; k > 0; k >>= 1) u += __shfl_down(u, k, 64);
        if (t == 0) *total = u;
    }
    __syncthreads();
    return *total;
}

// RMSNorm of one row of n: thread t adds x_i^2 for i = t, t + 256, ... (f64 fma), fixed tree,
// r = 1/sqrt(sum/n + eps), y_i = (x_i r) w_i in f64, rounded once (passe.cuh:235-259). x is read
// in full before the first write (y may be x). Up to NORME_PAR_FIL * 256 elements a thread holds
// its x and w values in registers, so all its loads go out together.
constexpr uint32_t NORME_PAR_FIL = 16;
__device__ __forceinline__ void norme_ligne(const float* __restrict__ x, const float* __restrict__ w, float* y,
                                            uint32_t n, float eps, double* part, double* total) {
    const uint32_t t = threadIdx.x;
    if (n <= NORME_PAR_FIL * FILS_NORME) {
        // indices clamped to the row (no branch around a load, so none waits for another); the
        // copies past the row are not used
        float xv[NORME_PAR_FIL], wv[NORME_PAR_FIL];
#pragma unroll
        for (uint32_t u = 0; u < NORME_PAR_FIL; ++u) {
            const uint32_t i = min(t + u * FILS_NORME, n - 1u);
            xv[u] = x[i];
            wv[u] = w[i];
        }
        double s = 0.0;
#pragma unroll
        for (uint32_t u = 0; u < NORME_PAR_FIL; ++u)
            if (t + u * FILS_NORME < n) s = fma(double(xv[u]), double(xv[u]), s);
        const double r = 1.0 / sqrt(somme_arbre_f64(part, total, s) / double(n) + double(eps));
#pragma unroll
        for (uint32_t u = 0; u < NORME_PAR_FIL; ++u) {
            const uint32_t i = t + u * FILS_NORME;
            if (i < n) y[i] = float(double(xv[u]) * r * double(wv[u]));
        }
        return;
    }
    double s = 0.0;
    for (uint32_t i = t; i < n; i += FILS_NORME) {
        const double v = x[i];
        s = fma(v, v, s);
    }
    const double r = 1.0 / sqrt(somme_arbre_f64(part, total, s) / double(n) + double(eps));
    for (uint32_t i = t; i < n; i += FILS_NORME) y[i] = float(double(x[i]) * r * double(w[i]));
}
}  // namespace trc
