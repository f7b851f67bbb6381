// fusion_corps.hpp — bodies of the fused-path kernels (gfx950): the DELTA pass that rebuilds the
// E8M0 scales, and the CODES_CTX pass that decodes the code bytes into registers and multiplies
// them against x on the fly.
//
// Mapping: one wavefront = two rANS tiles (lanes 0-31, 32-63), each tile's words staged in an LDS
// ring (anneau.hpp). In a macro-step, lane v of a tile produces the 4 code bytes 4(v%4) ..
// 4(v%4)+3 of block 8m + v/4, i.e. the weights of columns 32b + 4(v%4) + k (low nibbles) and
// 32b + 16 + 4(v%4) + k (high nibbles): two float4 of x. Each lane accumulates its block
// contributions per row; rows are closed by a 32-lane reduction when the tile's first block enters
// a new row (a row has >= 8 blocks, so one macro-step touches at most two rows). Every (row, tile)
// partial is written exactly once and summed in tile order by the finisher: results are
// deterministic, without floating-point atomics.
#pragma once

#include <type_traits>

#include "anneau.hpp"
#include "commun.hpp"

namespace trc {

// One job of the fused path: matrix j of a level-0 part, against x (48 bytes).
struct Tache {
    uint64_t partie;    // level-0 part
    uint64_t x;         // f32[colonnes], 16-byte aligned
    uint64_t ech;       // u8[lignes * colonnes/32] scales (workspace, 4-byte aligned)
    uint64_t partiels;  // f32[lignes * kmax] partial sums (workspace)
    uint32_t j;         // matrix index in the part
    uint32_t kmax;      // partial slots per row
    uint32_t lignes, colonnes;
};
static_assert(sizeof(Tache) == 48, "Tache");

// The jobs of a launch: a device table (MoE layer, built on the device) or up to 3 jobs passed by
// value in the kernel arguments (one matrix, one expert). Job of block (x, y) = y.
struct Taches {
    const Tache* table;
    Tache locales[3];
    __device__ __forceinline__ Tache operator[](uint32_t i) const { return table ? table[i] : locales[i]; }
};

constexpr uint32_t FILS_ECHELLES_FUSION = 256;  // 4 wavefronts, 8 DELTA tiles
constexpr uint32_t FILS_GEMV_FUSION = 1024;     // 16 wavefronts, 32 CODES_CTX tiles

__device__ __forceinline__ uint32_t premiere_tuile(uint32_t ligne, uint32_t B, uint32_t blocs_par_tuile) {
    return (ligne * B) / blocs_par_tuile;
}

template <typename T>
__device__ __forceinline__ void ecrire_global(void* p, T v) {
    *(__attribute__((address_space(1))) T*)(p) = v;
}

// ----------------------------------------------------------------------- DELTA -> scales only
__device__ __forceinline__ void corps_echelles_fusion(const Tache& tc, const uint2* lut, uint8_t* med_lds,
                                                      uint8_t* anneaux, uint32_t* __restrict__ controle) {
    const uint8_t* partie = reinterpret_cast<const uint8_t*>(tc.partie);
    const uint32_t R = tc.lignes, C = tc.colonnes, B = C / 32u, nblocs = R * B;
    DescFlux fd, fm;
    EnteteRans h;
    const bool bon = (C % 32u == 0) && B > 0 && R > 0 && trouver_flux(partie, SORTE_DELTA, tc.j, fd) &&
                     trouver_flux(partie, SORTE_MEDIANES, tc.j, fm) && fm.produits == R && fm.longueur >= R &&
                     lire_entete(fd, nblocs, h);
    if (!bon) {
        if (threadIdx.x == 0 && blockIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    const uint8_t* med = fm.p;
    if (R <= 8192u) {
        for (uint32_t i = threadIdx.x; i < R; i += blockDim.x) med_lds[i] = glob<uint8_t>(fm.p)[i];
        med = med_lds;
    }
    __syncthreads();
    uint8_t* ech = reinterpret_cast<uint8_t*>(tc.ech);
    const uint32_t lane = __lane_id();
    const uint32_t v = lane & 31u;
    const bool haut = lane >= 32u;
    const uint32_t decal = haut ? 32u : 0u, masque_inf = (1u << v) - 1u;
    const uint32_t vagues_bloc = blockDim.x >> 6;
    const uint32_t vague = blockIdx.x * vagues_bloc + (threadIdx.x >> 6);
    const uint32_t n_vagues = gridDim.x * vagues_bloc;
    const uint32_t lds = ((threadIdx.x >> 5) & (2u * vagues_bloc - 1u)) * OCTETS_ANNEAU;
    const uint32_t nmacro = h.P / 128u;
    uint32_t hors_l = 0, pointeur = 0;
    for (uint32_t t0 = 2u * vague; t0 < h.T; t0 += 2u * n_vagues) {
        const uint32_t t = t0 + (haut ? 1u : 0u);
        const bool tuile = t < h.T;
        const uint32_t nb_a = min(h.N, nmacro - t0 * h.N);
        const uint32_t nb_b = (t0 + 1u < h.T) ? min(h.N, nmacro - (t0 + 1u) * h.N) : 0u;
        const uint32_t nb = haut ? nb_b : nb_a;
        uint32_t x = tuile ? h.etats[t * VOIES + v] : L;
        const uint32_t debut = tuile ? h.debut[t] : 0u;
        Anneau a = ouvrir_anneau(h, fd, debut, lds, anneaux, v, tuile);
        const uint32_t o0 = a.o2;
        uint32_t b0 = 4u * ((tuile ? t : t0) * h.N * VOIES + v);
        uint32_t ligne = b0 / B, reste = b0 - ligne * B;
        auto macro = [&](auto tous, uint32_t m) {
            constexpr bool TOUS = decltype(tous)::value;
            const bool actif = TOUS || m < nb;
            uint32_t mot = 0;
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k)
                mot |= (pas_anneau<TOUS>(x, a, lut, anneaux, decal, masque_inf, actif) >> 24) << (8u * k);
            avancer_anneau(a, anneaux, v, actif);
            if (actif) {
                uint32_t sortie = 0;
#pragma unroll
                for (uint32_t k = 0; k < 4; ++k) {
                    uint32_t rk = ligne, qk = reste + k;
                    while (qk >= B) {
                        qk -= B;
                        ++rk;
                    }
                    const uint32_t mk = rk < R ? uint32_t(med[rk]) : 0u;
                    sortie |= ((mk + ((mot >> (8u * k)) & 255u) - 128u) & 255u) << (8u * k);
                }
                if (b0 + 3u < nblocs) {
                    ecrire_global<uint32_t>(ech + b0, sortie);
                } else {
                    for (uint32_t k = 0; k < 4; ++k)
                        if (b0 + k < nblocs) ecrire_global<uint8_t>(ech + b0 + k, uint8_t(sortie >> (8u * k)));
                }
            }
            b0 += 4u * VOIES;
            reste += 4u * VOIES;
            while (reste >= B) {
                reste -= B;
                ++ligne;
            }
        };
        const uint32_t nb_min = min(nb_a, nb_b);
        uint32_t m = 0;
        for (; m < nb_min; ++m) macro(std::true_type{}, m);
        for (; m < nb_a; ++m) macro(std::false_type{}, m);
        if (tuile) {
            hors_l += (x != L) ? 1u : 0u;
            const uint32_t attendu = (t + 1 < h.T) ? h.debut[t + 1] : h.W;
            pointeur += (v == 0 && debut + (a.o2 - o0) / 2u != attendu) ? 1u : 0u;
        }
    }
    verser_controle(controle, hors_l, pointeur);
}

// ------------------------------------------------------------ CODES_CTX -> partial sums of W x
__device__ __forceinline__ void corps_gemv_fusion(const Tache& tc, const uint2* lut, uint8_t* anneaux,
                                                  uint32_t* __restrict__ controle) {
    const uint8_t* partie = reinterpret_cast<const uint8_t*>(tc.partie);
    const uint32_t R = tc.lignes, C = tc.colonnes, B = C / 32u, nblocs = R * B;
    DescFlux fc, fm;
    EnteteRans h;
    bool bon = (C % 32u == 0) && B >= 8u && R > 0 && trouver_flux(partie, SORTE_CODES_CTX, tc.j, fc) &&
               trouver_flux(partie, SORTE_MEDIANES, tc.j, fm) && fm.produits == R && fm.longueur >= R &&
               lire_entete(fc, nblocs * 16u, h);
    if (bon && (B - 1u) / (8u * h.N) + 2u > tc.kmax) bon = false;  // not enough partial slots
    if (!bon) {
        if (threadIdx.x == 0 && blockIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    const gptr<uint8_t> med = glob<uint8_t>(fm.p);
    const gptr<uint8_t> ech = glob<uint8_t>(reinterpret_cast<const void*>(tc.ech));
    const gptr<f32x4> x4 = glob<f32x4>(reinterpret_cast<const void*>(tc.x));
    float* __restrict__ partiels = reinterpret_cast<float*>(tc.partiels);
    const uint32_t kmax = tc.kmax;
    const uint32_t bpt = 8u * h.N;  // blocks per tile

    const uint32_t lane = __lane_id();
    const uint32_t v = lane & 31u;
    const bool haut = lane >= 32u;
    const uint32_t decal = haut ? 32u : 0u, masque_inf = (1u << v) - 1u;
    const uint32_t q = v >> 2, q4 = v & 3u;
    const uint32_t vagues_bloc = blockDim.x >> 6;
    const uint32_t vague = blockIdx.x * vagues_bloc + (threadIdx.x >> 6);
    const uint32_t n_vagues = gridDim.x * vagues_bloc;
    const uint32_t lds = ((threadIdx.x >> 5) & (2u * vagues_bloc - 1u)) * OCTETS_ANNEAU;
    const uint32_t nmacro = h.P / 128u;
    uint32_t hors_l = 0, pointeur = 0;
    for (uint32_t t0 = 2u * vague; t0 < h.T; t0 += 2u * n_vagues) {
        const uint32_t t = t0 + (haut ? 1u : 0u);
        const bool tuile = t < h.T;
        const uint32_t nb_a = min(h.N, nmacro - t0 * h.N);
        const uint32_t nb_b = (t0 + 1u < h.T) ? min(h.N, nmacro - (t0 + 1u) * h.N) : 0u;
        const uint32_t nb = haut ? nb_b : nb_a;
        uint32_t x = tuile ? h.etats[t * VOIES + v] : L;
        const uint32_t debut = tuile ? h.debut[t] : 0u;
        Anneau a = ouvrir_anneau(h, fc, debut, lds, anneaux, v, tuile);
        const uint32_t o0 = a.o2;
        const uint32_t m0 = (tuile ? t : t0) * h.N;
        uint32_t bloc = m0 * 8u + q;
        uint32_t ligne = bloc / B, b = bloc - ligne * B;
        uint32_t rho = (m0 * 8u) / B, base_b = m0 * 8u - rho * B;  // row of the tile's first block
        bool valide = tuile && bloc < nblocs;
        uint32_t e_suiv = valide ? uint32_t(ech[bloc]) : 0u;
        uint32_t m_suiv = valide ? uint32_t(med[ligne]) : 0u;
        float acc_a = 0.0f, acc_b = 0.0f;
        auto macro = [&](auto tous, uint32_t m) {
            constexpr bool TOUS = decltype(tous)::value;
            const bool actif = TOUS || m < nb;
            const bool bloc_ok = valide;
            const uint32_t e_cur = e_suiv;
            const uint32_t ctx = bloc_ok ? classe_echelle(e_suiv, m_suiv) : 0u;
            const uint32_t b_cur = b;
            const bool ligne_a = ligne == rho;
            bloc += 8u;
            b += 8u;
            if (b >= B) {  // B >= 8: at most one row per macro-step
                b -= B;
                ++ligne;
            }
            valide = (m + 1u < nb) && bloc < nblocs;
            if (valide) {
                e_suiv = ech[bloc];
                m_suiv = med[ligne];
            }
            f32x4 xa = {0.f, 0.f, 0.f, 0.f}, xb = xa;
            if (bloc_ok) {
                xa = x4[8u * b_cur + q4];
                xb = x4[8u * b_cur + 4u + q4];
            }
            const uint2* lt = lut + ctx * M;
            const uint32_t e0 = pas_anneau<TOUS>(x, a, lt, anneaux, decal, masque_inf, actif);
            const uint32_t e1 = pas_anneau<TOUS>(x, a, lt, anneaux, decal, masque_inf, actif);
            const uint32_t e2 = pas_anneau<TOUS>(x, a, lt, anneaux, decal, masque_inf, actif);
            const uint32_t e3 = pas_anneau<TOUS>(x, a, lt, anneaux, decal, masque_inf, actif);
            avancer_anneau(a, anneaux, v, actif);
            if (actif && bloc_ok) {
                // byte 3 of each LUT word is the decoded code byte: two E2M1 values, doubled by
                // the 2.0 scale into the reference's k = {0,1,2,3,4,6,8,12} (exact)
                const f32x2 w0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e0, 2.0f, 3);
                const f32x2 w1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e1, 2.0f, 3);
                const f32x2 w2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e2, 2.0f, 3);
                const f32x2 w3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e3, 2.0f, 3);
                float d = w0.x * xa.x;
                d = fmaf(w0.y, xb.x, d);
                d = fmaf(w1.x, xa.y, d);
                d = fmaf(w1.y, xb.y, d);
                d = fmaf(w2.x, xa.z, d);
                d = fmaf(w2.y, xb.z, d);
                d = fmaf(w3.x, xa.w, d);
                d = fmaf(w3.y, xb.w, d);
                const float c = d * echelle_e8m0(e_cur);
                if (ligne_a)
                    acc_a += c;
                else
                    acc_b += c;
            }
            base_b += 8u;
            bool avance = false;
            if (base_b >= B) {
                base_b -= B;
                avance = actif;
            }
            if (__builtin_amdgcn_ballot_w64(avance) != 0) {
                const float s = somme_demi_f32(acc_a);
                if (avance) {
                    if (v == 0 && rho < R) partiels[rho * kmax + (t - premiere_tuile(rho, B, bpt))] = s;
                    acc_a = acc_b;
                    acc_b = 0.0f;
                    ++rho;
                }
            }
        };
        const uint32_t nb_min = min(nb_a, nb_b);
        uint32_t m = 0;
        for (; m < nb_min; ++m) macro(std::true_type{}, m);
        for (; m < nb_a; ++m) macro(std::false_type{}, m);
        const float sa = somme_demi_f32(acc_a);
        const float sb = somme_demi_f32(acc_b);
        if (tuile) {
            if (v == 0) {
                const uint32_t fin = min((m0 + nb) * 8u, nblocs);
                const uint32_t derniere = (fin - 1u) / B;
                if (rho <= derniere && rho < R) partiels[rho * kmax + (t - premiere_tuile(rho, B, bpt))] = sa;
                if (rho + 1u <= derniere && rho + 1u < R)
                    partiels[(rho + 1u) * kmax + (t - premiere_tuile(rho + 1u, B, bpt))] = sb;
            }
            hors_l += (x != L) ? 1u : 0u;
            const uint32_t attendu = (t + 1 < h.T) ? h.debut[t + 1] : h.W;
            pointeur += (v == 0 && debut + (a.o2 - o0) / 2u != attendu) ? 1u : 0u;
        }
    }
    verser_controle(controle, hors_l, pointeur);
}

}  // namespace trc
