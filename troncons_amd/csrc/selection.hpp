// selection.hpp — the router's top-k with softmax weights, as one wavefront's device function
// (shared by the reference-API kernel routeur_topk and the fused MoE layer).
//
// Order and arithmetic of the reference (passe.cuh:455-514): experts ranked by (logit desc, index
// asc); weights = softmax of the k chosen logits in f64 (m = the first, exp, sum in rank order,
// division), each rounded once to f32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace trc {

constexpr uint32_t TOPK_MAX = 8;
constexpr uint32_t EXPERTS_MAX = 256;

__device__ __forceinline__ bool meilleur(float va, uint32_t ia, float vb, uint32_t ib) {
    return va > vb || (va == vb && ia < ib);
}

// Executed by one whole wavefront (64 lanes, uniform E <= 256 and 1 <= k <= 8); every lane gets
// the same indices and weights.
__device__ __forceinline__ void topk_vague(const float* logits, uint32_t E, uint32_t k, uint32_t (&indice)[TOPK_MAX],
                                           float (&poids)[TOPK_MAX]) {
    const uint32_t voie = __lane_id();
    float v[4];
    bool pris[4];
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t e = voie + 64u * i;
        v[i] = e < E ? logits[e] : -INFINITY;
        pris[i] = e >= E;
    }
    float choisi[TOPK_MAX];
#pragma unroll
    for (uint32_t r = 0; r < TOPK_MAX; ++r) {
        choisi[r] = -INFINITY;
        indice[r] = 0xFFFFFFFFu;
        if (r < k) {
            float bv = -INFINITY;
            uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i)
                if (!pris[i] && meilleur(v[i], voie + 64u * i, bv, bi)) {
                    bv = v[i];
                    bi = voie + 64u * i;
                }
#pragma unroll
            for (int d = 32; d > 0; d >>= 1) {
                const float ov = __shfl_xor(bv, d);
                const uint32_t oi = __shfl_xor(bi, d);
                if (meilleur(ov, oi, bv, bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
#pragma unroll
            for (uint32_t i = 0; i < 4; ++i)
                if (bi == voie + 64u * i) pris[i] = true;
            choisi[r] = bv;
            indice[r] = bi;
        }
    }
    double e[TOPK_MAX];
    const double m = choisi[0];
    double z = 0.0;
#pragma unroll
    for (uint32_t r = 0; r < TOPK_MAX; ++r) {
        e[r] = 0.0;
        if (r < k) {
            e[r] = exp(double(choisi[r]) - m);
            z += e[r];
        }
    }
#pragma unroll
    for (uint32_t r = 0; r < TOPK_MAX; ++r) poids[r] = r < k ? float(e[r] / z) : 0.0f;
}

// Block-wide top-k by ranks (the selection of topk_vague without its serial rounds): the rank of
// expert i is the number of experts ordered before it by (logit desc, index asc); the expert of
// rank r < k is the r-th chosen. A NaN logit is never before another and is never chosen; slots
// past the number of non-NaN logits keep 0xFFFFFFFF, as in topk_vague.
// Each expert gets a group of `par` consecutive lanes (par a power of two, at most 64, par * E at
// most the block when it can be): lane c of the group counts over its share of the experts, the
// group adds its counts with lane exchanges, and its first lane writes the choice. No division,
// no LDS atomics. lg[0..E) in LDS (16-byte aligned) and choisis[0..TOPK_MAX) set to 0xFFFFFFFF
// before the call, barrier after it. fils: the block's thread count (a constant where the caller
// has one, so that it is not read from the dispatch packet).
__device__ __forceinline__ void choisir_topk(const float* lg, uint32_t E, uint32_t k, uint32_t* choisis,
                                             uint32_t fils) {
    uint32_t lpar = 0;
    while (lpar < 6u && (E << (lpar + 1u)) <= fils) ++lpar;
    const uint32_t par = 1u << lpar;
    const uint32_t part = (E + par - 1u) >> lpar;  // experts counted per lane
    const bool quatre = (part & 3u) == 0u && (E & 3u) == 0u;  // lanes' shares in whole 16-byte groups
    // every lane of a group takes the same trips: the exchanges below see only active lanes
    for (uint32_t q0 = threadIdx.x & ~(par - 1u); q0 < (E << lpar); q0 += fils) {
        const uint32_t q = q0 + (threadIdx.x & (par - 1u));
        const uint32_t i = q >> lpar, c = q & (par - 1u);
        const float vi = lg[i];
        const uint32_t j0 = c * part, j1 = min(E, j0 + part);
        uint32_t n = 0;
        if (quatre) {
            // 16-byte reads, four in flight: the counts do not wait on one LDS read after another
#pragma unroll 4
            for (uint32_t j = j0; j < j1; j += 4u) {
                const float4 w = *reinterpret_cast<const float4*>(lg + j);
                n += (w.x > vi || (w.x == vi && j < i)) ? 1u : 0u;
                n += (w.y > vi || (w.y == vi && j + 1u < i)) ? 1u : 0u;
                n += (w.z > vi || (w.z == vi && j + 2u < i)) ? 1u : 0u;
                n += (w.w > vi || (w.w == vi && j + 3u < i)) ? 1u : 0u;
            }
        } else {
            for (uint32_t j = j0; j < j1; ++j) {
                const float vj = lg[j];
                n += (vj > vi || (vj == vi && j < i)) ? 1u : 0u;
            }
        }
        for (uint32_t d = 1; d < par; d <<= 1) n += uint32_t(__shfl_xor(int(n), int(d)));
        if (c == 0u && vi == vi && n < k) choisis[n] = i;
    }
}

// The chosen experts' logits in rank order (-inf past k or past the non-NaN logits).
__device__ __forceinline__ void logits_choisis(const float* lg, const uint32_t* choisis, uint32_t k,
                                               float (&choisi)[TOPK_MAX]) {
#pragma unroll
    for (uint32_t r = 0; r < TOPK_MAX; ++r) choisi[r] = (r < k && choisis[r] != 0xFFFFFFFFu) ? lg[choisis[r]] : -INFINITY;
}

// The weights of topk_vague from the chosen experts' logits (same f64 softmax, one rounding each).
__device__ __forceinline__ void poids_de_logits(const float (&choisi)[TOPK_MAX], uint32_t k, float (&poids)[TOPK_MAX]) {
    double e[TOPK_MAX];
    const double m = choisi[0];
    double z = 0.0;
#pragma unroll
    for (uint32_t r = 0; r < TOPK_MAX; ++r) {
        e[r] = 0.0;
        if (r < k) {
            e[r] = exp(double(choisi[r]) - m);
            z += e[r];
        }
    }
#pragma unroll
    for (uint32_t r = 0; r < TOPK_MAX; ++r) poids[r] = r < k ? float(e[r] / z) : 0.0f;
}

__device__ __forceinline__ void poids_topk(const float* lg, const uint32_t* choisis, uint32_t k,
                                           float (&poids)[TOPK_MAX]) {
    float choisi[TOPK_MAX];
    logits_choisis(lg, choisis, k, choisi);
    poids_de_logits(choisi, k, poids);
}

}  // namespace trc
