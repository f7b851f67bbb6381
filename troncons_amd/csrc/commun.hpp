// commun.hpp — definitions shared by the host helpers and the gfx950 kernels of the expert hot path.
//
// Format facts restated from the reference's frozen seams (decisions/ARCHITECTURE.md §4.8-4.9, §5.6):
// the level-0 part (64-byte header, 16-byte stream descriptors), the rANS stream header
// (P, N, geometry, T, W, starts[T], states[32T], words[W]) and the SoA slot layout
// (codes, scales at al256(R*B*16), biases at al256(scales + R*B), stride al256(biases + 4R)).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/troncons_hip.h"

namespace trc {

constexpr uint32_t PROBA_BITS = 12;
constexpr uint32_t M = 1u << PROBA_BITS;  // 4096 slots
constexpr uint32_t L = 1u << 16;          // lower bound of a lane state
constexpr uint32_t VOIES = 32;            // lanes per tile
constexpr uint32_t MAGIE_PARTIE0 = 0x30435254u;  // "TRC0"

constexpr uint8_t SORTE_MEDIANES = 0x01;
constexpr uint8_t SORTE_BIAIS = 0x02;
constexpr uint8_t SORTE_DELTA = 0x03;
constexpr uint8_t SORTE_CODES_CTX = 0x04;
constexpr uint8_t SORTE_CODES_BRUTS = 0x06;
constexpr uint8_t SORTE_ECHELLES_BRUTES = 0x07;

// Control buffer slots (u32[4], zeroed by the caller).
constexpr int CTL_HORS_L = 0;
constexpr int CTL_FORMAT = 1;
constexpr int CTL_POINTEUR = 2;

// Threads per block of the reference-API kernels (abi.rs:56-61 keeps these a launch detail).
constexpr uint32_t FILS_ECHELLES = 128;  // 2 wavefronts = 4 DELTA tiles
constexpr uint32_t FILS_CODES = 256;     // 4 wavefronts = 8 CODES_CTX tiles
constexpr uint32_t FILS_BRUT = 256;
constexpr uint32_t GEMV_FILS = 256;
constexpr uint32_t GEMV_LIGNES_PAR_BLOC = 16;  // 8 half-wavefronts x 2 rows
constexpr uint32_t LUTS_PAR_COUCHE = 3 * 4 * 4096;
constexpr uint32_t MACRO_PAR_TUILE = 256;  // what the reference encoder writes; used for grids only

__host__ __device__ inline uint64_t al256(uint64_t x) { return (x + 255u) & ~uint64_t(255); }

__host__ __device__ inline trc_disposition disposition_matrice(uint32_t lignes, uint32_t colonnes) {
    const uint64_t blocs = uint64_t(lignes) * (colonnes / 32u);
    trc_disposition d;
    d.base = 0;
    d.echelles = al256(blocs * 16u);
    d.biais = al256(d.echelles + blocs);
    d.pas = al256(d.biais + 4ull * lignes);
    return d;
}

// Element j of a 3-array without a dynamic index (a dynamic index would spill it to scratch).
__host__ __device__ __forceinline__ uint32_t choisir(const uint32_t (&a)[3], uint32_t j) {
    return j == 0 ? a[0] : (j == 1 ? a[1] : a[2]);
}

__host__ __device__ inline trc_disposition disposition(const trc_dims_expert& dims, uint32_t j) {
    uint64_t base = 0;
#pragma unroll
    for (uint32_t i = 0; i < 3; ++i)
        if (i < j) base += disposition_matrice(dims.lignes[i], dims.colonnes[i]).pas;
    trc_disposition d = disposition_matrice(choisir(dims.lignes, j), choisir(dims.colonnes, j));
    d.base = base;
    return d;
}

// ------------------------------------------------------------------------- device-side part reading

// Global-address-space views: loads through them compile to global_load (vmcnt only) instead of
// flat_load (which also counts in lgkmcnt and would make every LDS wait wait for them too).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <typename T>
using gptr = __attribute__((address_space(1))) const T*;
template <typename T>
__device__ __forceinline__ gptr<T> glob(const void* p) {
    return (gptr<T>)(p);
}

struct DescFlux {
    const uint8_t* p;
    uint32_t longueur;
    uint32_t produits;
};

// Finds streams (sortes[i], matrice) for i < n (n <= 4) of a level-0 part in one pass over its
// descriptors, with the acceptance of the reference device reader (commun.cuh:111-129): for each
// kind the first matching descriptor, whose offset is 16-aligned and whose bytes lie inside the part.
// False if the part is malformed or a stream is absent. The part must be 16-byte aligned. Executed
// by a whole wavefront with uniform arguments: lane i loads descriptor i (a part has at most 64),
// one ballot per kind finds the first match.
__device__ inline bool trouver_flux_n(const uint8_t* partie, const uint8_t (&sortes)[4], uint32_t n, uint32_t matrice,
                                      DescFlux (&f)[4]) {
    if (partie == nullptr || (reinterpret_cast<uintptr_t>(partie) & 15u) != 0) return false;
    const u32x4 en = *glob<u32x4>(partie);
    const uint32_t n_flux = en.z >> 16, utiles = en.w;
    if (en.x != MAGIE_PARTIE0 || (en.z & 0xFFu) != 0) return false;
    if (n_flux > 64 || 64u + 16u * n_flux > utiles) return false;
    const uint32_t lane = __lane_id();
    u32x4 d = {0u, 0u, 0u, 0u};
    if (lane < n_flux) d = *glob<u32x4>(partie + 64 + 16 * lane);
    bool tous = true;
#pragma unroll
    for (uint32_t s = 0; s < 4; ++s) {
        if (s >= n) break;
        const bool ok = lane < n_flux && (d.x & 0xFFu) == sortes[s] && ((d.x >> 8) & 0xFFu) == matrice;
        const uint64_t vote = __builtin_amdgcn_ballot_w64(ok);
        if (vote == 0) {
            tous = false;
            continue;
        }
        const uint32_t i = uint32_t(__builtin_ctzll(vote));
        const uint32_t dec = uint32_t(__builtin_amdgcn_readlane(d.y, i));
        const uint32_t lon = uint32_t(__builtin_amdgcn_readlane(d.z, i));
        if ((dec & 15u) != 0 || uint64_t(dec) + lon > utiles) tous = false;
        f[s].p = partie + dec;
        f[s].longueur = lon;
        f[s].produits = uint32_t(__builtin_amdgcn_readlane(d.w, i));
    }
    return tous;
}

// A validated rANS stream header (geometry 1).
struct EnteteRans {
    uint32_t P, N, T, W;
    const uint32_t* debut;   // T word indices
    const uint32_t* etats;   // 32*T lane states
    const uint16_t* mots;    // W 16-bit words
};

// `besoin`: bytes the caller needs; the stream produces P >= besoin with less than 128 bytes of
// padding, and its descriptor announces P or besoin (commun.cuh:143-165).
__device__ inline bool lire_entete(const DescFlux& f, uint32_t besoin, EnteteRans& h) {
    if (f.longueur < 16) return false;
    const u32x4 en = *glob<u32x4>(f.p);  // streams are 16-byte aligned in their part
    h.P = en.x;
    h.N = en.y & 0xFFFFu;
    const uint32_t geo = (en.y >> 16) & 0xFFu;
    h.T = en.z;
    h.W = en.w;
    if (geo != 1 || h.N == 0 || (h.P & 127u) != 0) return false;
    if (h.P < besoin || h.P - besoin >= 128u) return false;
    if (f.produits != h.P && f.produits != besoin) return false;
    const uint32_t macro = h.P / 128u;
    if (h.T != (macro + h.N - 1) / h.N) return false;
    const uint64_t fin = 16ull + 132ull * h.T + 2ull * h.W;
    if (fin > f.longueur) return false;
    h.debut = reinterpret_cast<const uint32_t*>(f.p + 16);
    h.etats = reinterpret_cast<const uint32_t*>(f.p + 16 + 4ull * h.T);
    h.mots = reinterpret_cast<const uint16_t*>(f.p + 16 + 132ull * h.T);
    return true;
}

// The header of an already validated stream from its fields.
__device__ __forceinline__ EnteteRans entete_de(const DescFlux& f, uint32_t P, uint32_t N, uint32_t T, uint32_t W) {
    EnteteRans h;
    h.P = P;
    h.N = N;
    h.T = T;
    h.W = W;
    h.debut = reinterpret_cast<const uint32_t*>(f.p + 16);
    h.etats = reinterpret_cast<const uint32_t*>(f.p + 16 + 4ull * T);
    h.mots = reinterpret_cast<const uint16_t*>(f.p + 16 + 132ull * T);
    return h;
}

// Scale class kappa of a block from its scale e and its row median (delta = e - med + 128 mod 256).
__device__ __forceinline__ uint32_t classe_echelle(uint32_t e, uint32_t med) {
    const uint32_t delta = (e - med + 128u) & 255u;
    return delta < 128u ? 0u : (delta == 128u ? 1u : 2u);
}

// Integer wave sum, fixed tree (exact and deterministic).
__device__ __forceinline__ uint32_t somme_vague_u32(uint32_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d);
    return v;
}

__device__ __forceinline__ void verser_controle(uint32_t* controle, uint32_t hors_l, uint32_t pointeur) {
    if (__builtin_amdgcn_ballot_w64((hors_l | pointeur) != 0u) == 0) return;  // the usual case: nothing to count
    hors_l = somme_vague_u32(hors_l);
    pointeur = somme_vague_u32(pointeur);
    if (__lane_id() == 0) {
        if (hors_l) atomicAdd(&controle[CTL_HORS_L], hors_l);
        if (pointeur) atomicAdd(&controle[CTL_POINTEUR], pointeur);
    }
}

// 32-lane xor butterfly within each half-wavefront (the reference's warp reduction tree).
__device__ __forceinline__ float somme_demi_f32(float v) {
#pragma unroll
    for (int d = 16; d > 0; d >>= 1) v += __shfl_xor(v, d);
    return v;
}

// 2^(e-128) in f32, exact for every e (e = 0, 1 are subnormal).
__device__ __forceinline__ float echelle_e8m0(uint32_t e) {
    const uint32_t bits = e >= 2u ? (e - 1u) << 23 : (0x00200000u << e);
    return __uint_as_float(bits);
}

}  // namespace trc
