// emplacement.hpp — the slot decoders' bodies (gfx950): DELTA -> E8M0 scales and biases, then
// CODES_CTX -> code bytes, written into the reference's SoA slot (commun.cuh:49-92, abi.rs:76-122).
// Shared by the reference-API kernels (noyaux.hip: decoder_echelles / decoder_codes and their batch
// forms, streams located in the part) and the batched prefill of long tiles (prefill.hip: streams
// taken from the mounted layer's directory).
#pragma once

#include "anneau.hpp"
#include "commun.hpp"
#include "entiers.hpp"
#include "fusion_corps.hpp"

namespace trc {

// ================================================================= slot decoders (gfx950 engine)
//
// Both decoders run the fused path's rANS engine (anneau.hpp): two tiles per wavefront (one per
// 32-lane half), the tile's words staged in a 1 KiB LDS ring refilled one macro-step ahead, the
// LUT re-expanded in LDS to 8-byte entries {f | s << 24, b} so a step is one v_mad_u32_u24.
// Only the consumer differs from the fused passes: a macro-step's 4 bytes per lane are stored into
// the slot instead of being multiplied against x.
//
// Lane v of a tile's half, in the tile's macro-step m (global macro-step g = t * N + m), decodes
// word w = 32 g + v: for DELTA the deltas of blocks 4w .. 4w + 3, for CODES_CTX code bytes
// 4w .. 4w + 3 of block w / 4. A block's row is block / B (B blocks per row), computed with a
// multiply-high (Diviseur).

// The half-wavefront's tile geometry and its end checks.
struct Demi {
    uint32_t v, decal, masque_inf, demi;  // lane in the half, its ballot shift, lower lanes, half index in the block
    bool haut;
};
__device__ __forceinline__ Demi demi_courante() {
    Demi d;
    const uint32_t lane = __lane_id();
    d.v = lane & 31u;
    d.haut = lane >= 32u;
    d.decal = d.haut ? 32u : 0u;
    d.masque_inf = (1u << d.v) - 1u;
    d.demi = threadIdx.x >> 5;
    return d;
}

// End-of-tile checks (commun.cuh:197-218 semantics): every lane back at L, and the words consumed
// ending exactly where the next tile's words start (or at W for the last tile).
__device__ __forceinline__ void verifier_tuile(const EnteteRans& h, uint32_t t, uint32_t x, uint32_t debut,
                                               uint32_t consommes, uint32_t v, uint32_t& hors_l, uint32_t& pointeur) {
    hors_l += (x != L) ? 1u : 0u;
    const uint32_t attendu = (t + 1u < h.T) ? h.debut[t + 1u] : h.W;
    pointeur += (v == 0u && debut + consommes != attendu) ? 1u : 0u;
}

// Biases: a bit copy (as u32, so no conversion ever touches a NaN), 16 bytes at a time where both
// sides allow it. Spread over the grid's x dimension.
__device__ __forceinline__ void copier_biais(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t R) {
    const uint32_t pas = gridDim.x * blockDim.x;
    const uint32_t n16 = R / 4u;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += pas)
        ecrire_global<u32x4>(dst + 16u * i, glob<u32x4>(src)[i]);
    for (uint32_t i = 4u * n16 + blockIdx.x * blockDim.x + threadIdx.x; i < R; i += pas)
        ecrire_global<uint32_t>(dst + 4u * i, glob<uint32_t>(src)[i]);
}

// The decoded bytes (byte 3 of each LUT word of a macro-step's four steps) as one word, step k in
// byte k: two byte permutes and an or.
__device__ __forceinline__ uint32_t octets_hauts(uint32_t e0, uint32_t e1, uint32_t e2, uint32_t e3) {
    return __builtin_amdgcn_perm(e1, e0, 0x0c0c0703u) | __builtin_amdgcn_perm(e3, e2, 0x07030c0cu);
}

template <uint32_t FILS>
struct LdsEchelles {
    uint2 lut[M];
    __attribute__((aligned(OCTETS_ANNEAU))) uint8_t anneaux[(FILS / 32u) * OCTETS_ANNEAU];
    __attribute__((aligned(16))) uint8_t med[MED_LDS_MAX];
};

// ----------------------------------------------------------------- DELTA -> E8M0 scales of the slot
// e(block) = (med[row] + delta - 128) mod 256 (rans.rs:231-280); biases copied bit for bit.
// The body, over located streams: fd (DELTA, header h), fm (MEDIANES), fb (BIAIS) of matrix j
// (R rows of B blocks), already checked; mat = the matrix's place in the slot (layout disp). Tiles
// go to the grid's x dimension (blockIdx.y = j).
template <uint32_t FILS>
__device__ __forceinline__ void echelles_vers_emplacement(const DescFlux& fd, const DescFlux& fm, const DescFlux& fb,
                                                          const EnteteRans& h, uint32_t R, uint32_t B, uint8_t* mat,
                                                          const trc_disposition& disp, const uint32_t* __restrict__ lutd,
                                                          uint32_t* __restrict__ controle, LdsEchelles<FILS>& s) {
    const uint32_t nblocs = R * B;
    copier_biais(fb.p, mat + disp.biais, R);
    etendre_luts<(M / 4u + FILS - 1u) / FILS>(lutd, s.lut, M / 4u);
    const uint8_t* med = fm.p;
    if (R <= MED_LDS_MAX) {
        copier_vers_lds(fm.p, R, fm.longueur, s.med);
        med = s.med;
    }
    __syncthreads();

    const Demi d = demi_courante();
    const Diviseur parB = Diviseur::de(B);
    const uint32_t vague = blockIdx.x * (FILS / 64u) + (threadIdx.x >> 6), n_vagues = gridDim.x * (FILS / 64u);
    const uint32_t nmacro = h.P / 128u;
    const uint32_t a_lut = adresse_lds(&s.lut[0]);
    const uint32_t a_anneau = adresse_lds(s.anneaux) + d.demi * OCTETS_ANNEAU;
    uint8_t* ech = mat + disp.echelles;
    uint32_t hors_l = 0, pointeur = 0;
    for (uint32_t t0 = 2u * vague; t0 < h.T; t0 += 2u * n_vagues) {
        const uint32_t t = t0 + (d.haut ? 1u : 0u);
        const bool tuile = t < h.T;
        const uint32_t pas_bas = min(h.N, nmacro - t0 * h.N);  // the lower tile is never the shorter one
        const uint32_t nb = tuile ? min(h.N, nmacro - t * h.N) : 0u;
        uint32_t x = tuile ? h.etats[t * VOIES + d.v] : L;
        const uint32_t debut = tuile ? h.debut[t] : 0u;
        AnneauR a = ouvrir_anneau_r(h, fd, debut, a_anneau, d.v, tuile);
        const uint32_t o0 = a.o2;
        // macro-steps where both tiles of the wavefront are active take the branch-free step
        const uint32_t n_tous = t0 + 1u < h.T ? min(pas_bas, min(h.N, nmacro - (t0 + 1u) * h.N)) : 0u;
        auto macro = [&](auto tous, uint32_t m) {
            constexpr bool TOUS = decltype(tous)::value;
            const bool actif = TOUS || m < nb;
            uint32_t compte = 0;
            const uint32_t e0 = pas_r<TOUS>(x, a.o2, compte, a_lut, a_anneau, d.decal, d.masque_inf, actif);
            const uint32_t e1 = pas_r<TOUS>(x, a.o2, compte, a_lut, a_anneau, d.decal, d.masque_inf, actif);
            const uint32_t e2 = pas_r<TOUS>(x, a.o2, compte, a_lut, a_anneau, d.decal, d.masque_inf, actif);
            const uint32_t e3 = pas_r<TOUS>(x, a.o2, compte, a_lut, a_anneau, d.decal, d.masque_inf, actif);
            a.o2 += 2u * compte;
            avancer_anneau_r(a, d.v, actif);
            const uint32_t deltas = octets_hauts(e0, e1, e2, e3);
            const uint32_t b0 = 4u * ((t * h.N + m) * VOIES + d.v);
            if (!actif || b0 >= nblocs) return;  // stream padding past the last block
            const uint32_t r0 = parB.quotient(b0), c0 = b0 - r0 * B;
            uint32_t e4 = 0;
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) {
                const uint32_t r = c0 + k < B ? r0 : parB.quotient(b0 + k);
                const uint32_t mr = r < R ? uint32_t(med[r]) : 0u;
                e4 |= ((mr + ((deltas >> (8u * k)) & 255u) - 128u) & 255u) << (8u * k);
            }
            if (b0 + 4u <= nblocs) {
                ecrire_global<uint32_t>(ech + b0, e4);  // b0 % 4 == 0 and the scales are 256-aligned
            } else {
                for (uint32_t k = 0; b0 + k < nblocs; ++k) ecrire_global<uint8_t>(ech + b0 + k, uint8_t(e4 >> (8u * k)));
            }
        };
        uint32_t m = 0;
        for (; m < n_tous; ++m) macro(std::true_type{}, m);
        for (; m < pas_bas; ++m) macro(std::false_type{}, m);
        if (tuile) verifier_tuile(h, t, x, debut, (a.o2 - o0) / 2u, d.v, hors_l, pointeur);
    }
    verser_controle(controle, hors_l, pointeur);
}

// From a part: matrix j = blockIdx.y located in its stream table and checked as the reference's
// device reader does.
template <uint32_t FILS>
__device__ __forceinline__ void decoder_echelles_corps(const uint8_t* __restrict__ partie, uint8_t* __restrict__ emplacement,
                                                      const uint32_t* __restrict__ luts, const trc_dims_expert& dims,
                                                      uint32_t* __restrict__ controle, LdsEchelles<FILS>& s) {
    const uint32_t j = blockIdx.y;
    const uint32_t R = choisir(dims.lignes, j), C = choisir(dims.colonnes, j);
    const uint32_t B = C / 32u, nblocs = R * B;
    constexpr uint8_t sortes[4] = {SORTE_DELTA, SORTE_MEDIANES, SORTE_BIAIS, 0};
    DescFlux f[4];
    EnteteRans h;
    const bool bon = C % 32u == 0 && B > 0 && R > 0 && trouver_flux_n(partie, sortes, 3, j, f) && f[1].produits == R &&
                     f[1].longueur >= R && f[2].produits == 4u * R && f[2].longueur >= 4u * R &&
                     lire_entete(f[0], nblocs, h);
    if (!bon) {  // uniform over the block: every thread leaves here
        if (threadIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    const trc_disposition disp = disposition(dims, j);
    echelles_vers_emplacement<FILS>(f[0], f[1], f[2], h, R, B, emplacement + disp.base, disp, luts + uint64_t(j) * 4u * M,
                                    controle, s);
}

// ------------------------------------------------------------ CODES_CTX -> code words of the slot
// The context of block b is the class of delta = e(b) - med[row] + 128 (decodeur.cuh:185-192),
// e(b) read back from the slot's scales (the DELTA decoder ran first on the same stream). Each half
// stages the contexts of 16 macro-steps (128 blocks, 4 per lane) in LDS at a time; the scale bytes
// of the next 16 are loaded one group ahead, so a group switch waits for nothing in the usual case.
constexpr uint32_t FILS_CODES_SLOT = FILS_CODES;
template <uint32_t FILS>
struct LdsCodesT {
    uint2 lut[3][M];
    __attribute__((aligned(OCTETS_ANNEAU))) uint8_t anneaux[(FILS / 32u) * OCTETS_ANNEAU];
    __attribute__((aligned(16))) uint8_t ctx[FILS / 32u][128];
    __attribute__((aligned(16))) uint8_t med[MED_LDS_MAX];
};
using LdsCodes = LdsCodesT<FILS_CODES_SLOT>;

// Scale bytes of blocks b0 .. b0 + 3 (b0 % 4 == 0), 0 past the matrix.
__device__ __forceinline__ uint32_t lire_echelles4(const uint8_t* ech, uint32_t b0, uint32_t nblocs) {
    if (b0 + 4u <= nblocs) return *glob<uint32_t>(ech + b0);
    uint32_t e4 = 0;
    for (uint32_t k = 0; b0 + k < nblocs && k < 4u; ++k) e4 |= uint32_t(glob<uint8_t>(ech)[b0 + k]) << (8u * k);
    return e4;
}

__device__ __forceinline__ uint32_t contextes4(uint32_t e4, uint32_t b0, uint32_t nblocs, const Diviseur& parB,
                                               uint32_t B, const uint8_t* med) {
    if (b0 >= nblocs) return 0u;
    const uint32_t r0 = parB.quotient(b0), c0 = b0 - r0 * B;
    uint32_t k4 = 0;
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
        if (b0 + k >= nblocs) break;
        const uint32_t r = c0 + k < B ? r0 : parB.quotient(b0 + k);
        k4 |= classe_echelle((e4 >> (8u * k)) & 255u, med[r]) << (8u * k);
    }
    return k4;
}

// The body, over located and checked streams: fc (CODES_CTX, header h) and fm (MEDIANES) of matrix
// j (R rows of B blocks); mat = the matrix's place in the slot, whose scales are already decoded;
// lutc = the matrix's three CODES_CTX tables (reference format).
template <uint32_t FILS>
__device__ __forceinline__ void codes_vers_emplacement(const DescFlux& fc, const DescFlux& fm, const EnteteRans& h,
                                                       uint32_t R, uint32_t B, uint8_t* mat, const trc_disposition& disp,
                                                       const uint32_t* __restrict__ lutc, uint32_t* __restrict__ controle,
                                                       LdsCodesT<FILS>& s) {
    const uint32_t nblocs = R * B;
    const uint8_t* ech = mat + disp.echelles;
    etendre_luts<(3u * M / 4u + FILS - 1u) / FILS>(lutc, &s.lut[0][0], 3u * M / 4u);
    const uint8_t* med = fm.p;
    if (R <= MED_LDS_MAX) {
        copier_vers_lds(fm.p, R, fm.longueur, s.med);
        med = s.med;
    }
    __syncthreads();

    const Demi d = demi_courante();
    const Diviseur parB = Diviseur::de(B);
    const uint32_t vague = blockIdx.x * (FILS / 64u) + (threadIdx.x >> 6), n_vagues = gridDim.x * (FILS / 64u);
    const uint32_t nmacro = h.P / 128u;
    const uint32_t mots_utiles = 4u * nblocs;
    const uint32_t a_ctx = adresse_lds(&s.ctx[d.demi][0]);
    const uint32_t a_lut = adresse_lds(&s.lut[0][0]);
    const uint32_t a_anneau = adresse_lds(s.anneaux) + d.demi * OCTETS_ANNEAU;
    uint32_t* codes = reinterpret_cast<uint32_t*>(mat);
    uint32_t hors_l = 0, pointeur = 0;
    for (uint32_t t0 = 2u * vague; t0 < h.T; t0 += 2u * n_vagues) {
        const uint32_t t = t0 + (d.haut ? 1u : 0u);
        const bool tuile = t < h.T;
        const uint32_t pas_bas = min(h.N, nmacro - t0 * h.N);
        const uint32_t nb = tuile ? min(h.N, nmacro - t * h.N) : 0u;
        const uint32_t g0 = (tuile ? t : t0) * h.N;  // the tile's first global macro-step
        uint32_t x = tuile ? h.etats[t * VOIES + d.v] : L;
        const uint32_t debut = tuile ? h.debut[t] : 0u;
        uint32_t e_vol = tuile ? lire_echelles4(ech, 8u * g0 + 4u * d.v, nblocs) : 0u;
        AnneauR a = ouvrir_anneau_r(h, fc, debut, a_anneau, d.v, tuile);
        const uint32_t o0 = a.o2;
        const uint32_t n_tous = t0 + 1u < h.T ? min(pas_bas, min(h.N, nmacro - (t0 + 1u) * h.N)) : 0u;
        auto macro = [&](auto tous, uint32_t m) {
            constexpr bool TOUS = decltype(tous)::value;
            const bool actif = TOUS || m < nb;
            if ((m & 15u) == 0u) {  // a new group of 16 macro-steps: its contexts into LDS, the next group's scales requested
                const uint32_t b0 = 8u * (g0 + m) + 4u * d.v;
                ecrire_lds<uint32_t>(a_ctx + 4u * d.v, actif ? contextes4(e_vol, b0, nblocs, parB, B, med) : 0u);
                if (m + 16u < nb) e_vol = lire_echelles4(ech, b0 + 128u, nblocs);
            }
            const uint32_t kappa = lire_lds<uint8_t>(a_ctx + 8u * (m & 15u) + (d.v >> 2));
            const uint32_t lt = a_lut + kappa * (M * 8u);
            uint32_t compte = 0;
            const uint32_t e0 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, d.decal, d.masque_inf, actif);
            const uint32_t e1 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, d.decal, d.masque_inf, actif);
            const uint32_t e2 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, d.decal, d.masque_inf, actif);
            const uint32_t e3 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, d.decal, d.masque_inf, actif);
            a.o2 += 2u * compte;
            avancer_anneau_r(a, d.v, actif);
            const uint32_t w = (g0 + m) * VOIES + d.v;
            if (actif && w < mots_utiles) ecrire_global<uint32_t>(codes + w, octets_hauts(e0, e1, e2, e3));
        };
        uint32_t m = 0;
        for (; m < n_tous; ++m) macro(std::true_type{}, m);
        for (; m < pas_bas; ++m) macro(std::false_type{}, m);
        if (tuile) verifier_tuile(h, t, x, debut, (a.o2 - o0) / 2u, d.v, hors_l, pointeur);
    }
    verser_controle(controle, hors_l, pointeur);
}

// From a part: matrix j = blockIdx.y located in its stream table and checked.
template <uint32_t FILS>
__device__ __forceinline__ void decoder_codes_corps(const uint8_t* __restrict__ partie, uint8_t* __restrict__ emplacement,
                                                   const uint32_t* __restrict__ luts, const trc_dims_expert& dims,
                                                   uint32_t* __restrict__ controle, LdsCodesT<FILS>& s) {
    const uint32_t j = blockIdx.y;
    const uint32_t R = choisir(dims.lignes, j), C = choisir(dims.colonnes, j);
    const uint32_t B = C / 32u, nblocs = R * B;
    constexpr uint8_t sortes[4] = {SORTE_CODES_CTX, SORTE_MEDIANES, 0, 0};
    DescFlux f[4];
    EnteteRans h;
    const bool bon = C % 32u == 0 && B > 0 && R > 0 && trouver_flux_n(partie, sortes, 2, j, f) && f[1].produits == R &&
                     f[1].longueur >= R && lire_entete(f[0], nblocs * 16u, h);
    if (!bon) {
        if (threadIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    const trc_disposition disp = disposition(dims, j);
    codes_vers_emplacement<FILS>(f[0], f[1], h, R, B, emplacement + disp.base, disp,
                                 luts + (uint64_t(j) * 4u + 1u) * M, controle, s);
}

}  // namespace trc
