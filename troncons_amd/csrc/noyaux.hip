// noyaux.hip — the reference kernel API of the expert hot path, written for gfx950.
//
// Same names, arguments and results as the reference's CUDA kernels (moteur/crates/trc-noyaux/
// noyaux/decodeur.cuh, gemv.cuh, passe.cuh) so that the engine's launch layer maps one to one;
// the bodies are wave64-native: a wavefront decodes two rANS tiles (one per 32-lane half), the
// LUTs sit in LDS, and the GEMV runs two reference "warps" per wavefront so that its operation
// order (and therefore every output bit) is the reference's.
//
// Determinism: no floating-point atomics; the only atomics are integer control counters.
#include <hip/hip_runtime.h>

#include "commun.hpp"
#include "erreurs.hpp"
#include "selection.hpp"

namespace trc {

// ===================================================================== decoder: DELTA -> scales
__device__ __forceinline__ void corps_echelles(const uint8_t* __restrict__ partie, uint8_t* __restrict__ emplacement,
                                               const uint32_t* __restrict__ luts, const trc_dims_expert& dims,
                                               uint32_t* __restrict__ controle, uint32_t* lut, uint8_t* med_lds) {
    const uint32_t j = blockIdx.y;
    const uint32_t* src = luts + (uint64_t(j) * 4u + 0u) * M;
    for (uint32_t i = threadIdx.x; i < M; i += blockDim.x) lut[i] = src[i];
    __syncthreads();

    const uint32_t R = choisir(dims.lignes, j), C = choisir(dims.colonnes, j);
    const uint32_t B = C / 32u, nblocs = R * B;
    DescFlux fd, fm, fb;
    EnteteRans h;
    const bool bon = (C % 32u == 0) && B > 0 && R > 0 && trouver_flux(partie, SORTE_DELTA, j, fd) &&
                     trouver_flux(partie, SORTE_MEDIANES, j, fm) && trouver_flux(partie, SORTE_BIAIS, j, fb) &&
                     fm.produits == R && fm.longueur >= R && fb.produits == 4u * R && fb.longueur >= 4u * R &&
                     lire_entete(fd, nblocs, h);
    if (!bon) {
        if (threadIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    const trc_disposition disp = disposition(dims, j);
    uint8_t* mat = emplacement + disp.base;
    {  // biases: bit copy (u32: no conversion touches a NaN)
        const uint32_t* bs = reinterpret_cast<const uint32_t*>(fb.p);
        uint32_t* bd = reinterpret_cast<uint32_t*>(mat + disp.biais);
        for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < R; i += gridDim.x * blockDim.x) bd[i] = bs[i];
    }
    const uint8_t* med = fm.p;
    if (R <= 8192u) {
        for (uint32_t i = threadIdx.x; i < R; i += blockDim.x) med_lds[i] = fm.p[i];
        med = med_lds;
    }
    __syncthreads();

    uint8_t* ech = mat + disp.echelles;
    const DemiVague dv = demi_vague();
    const uint32_t v = __lane_id() & 31u;
    const uint32_t vagues_bloc = blockDim.x >> 6;
    const uint32_t vague = blockIdx.x * vagues_bloc + (threadIdx.x >> 6);
    const uint32_t n_vagues = gridDim.x * vagues_bloc;
    const uint32_t nmacro = h.P / 128u;
    uint32_t hors_l = 0, pointeur = 0;
    for (uint32_t t0 = 2u * vague; t0 < h.T; t0 += 2u * n_vagues) {
        const uint32_t t = t0 + (dv.haut ? 1u : 0u);
        const bool tuile = t < h.T;
        const uint32_t nb_a = min(h.N, nmacro - t0 * h.N);
        const uint32_t nb = tuile ? min(h.N, nmacro - t * h.N) : 0u;
        uint32_t x = tuile ? h.etats[t * VOIES + v] : L;
        uint32_t ptr = tuile ? h.debut[t] : 0u;
        // word w = m*32 + v carries the deltas of blocks 4w .. 4w+3; row and remainder of 4w are
        // tracked without division (4w advances by 128 per macro-step).
        uint32_t b0 = 4u * ((tuile ? t : t0) * h.N * VOIES + v);
        uint32_t ligne = b0 / B, reste = b0 - ligne * B;
        for (uint32_t m = 0; m < nb_a; ++m) {
            const bool actif = m < nb;
            uint32_t mot = 0;
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) mot |= pas_octet(x, ptr, lut, h.mots, h.W, dv, actif) << (8u * k);
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
                    reinterpret_cast<uint32_t*>(ech)[b0 >> 2] = sortie;
                } else {
                    for (uint32_t k = 0; k < 4; ++k)
                        if (b0 + k < nblocs) ech[b0 + k] = uint8_t(sortie >> (8u * k));
                }
            }
            b0 += 4u * VOIES;
            reste += 4u * VOIES;
            while (reste >= B) {
                reste -= B;
                ++ligne;
            }
        }
        if (tuile) {
            hors_l += (x != L) ? 1u : 0u;
            const uint32_t attendu = (t + 1 < h.T) ? h.debut[t + 1] : h.W;
            pointeur += (v == 0 && ptr != attendu) ? 1u : 0u;
        }
    }
    verser_controle(controle, hors_l, pointeur);
}

// ============================================================== decoder: CODES_CTX -> code words
__device__ __forceinline__ void corps_codes(const uint8_t* __restrict__ partie, uint8_t* __restrict__ emplacement,
                                            const uint32_t* __restrict__ luts, const trc_dims_expert& dims,
                                            uint32_t* __restrict__ controle, uint32_t (*lut)[M]) {
    const uint32_t j = blockIdx.y;
    {
        const uint32_t* src = luts + (uint64_t(j) * 4u + 1u) * M;
        uint32_t* dst = &lut[0][0];
        for (uint32_t i = threadIdx.x; i < 3u * M; i += blockDim.x) dst[i] = src[i];
    }
    __syncthreads();

    const uint32_t R = choisir(dims.lignes, j), C = choisir(dims.colonnes, j);
    const uint32_t B = C / 32u, nblocs = R * B;
    DescFlux fc, fm;
    EnteteRans h;
    const bool bon = (C % 32u == 0) && B > 0 && R > 0 && trouver_flux(partie, SORTE_CODES_CTX, j, fc) &&
                     trouver_flux(partie, SORTE_MEDIANES, j, fm) && fm.produits == R && fm.longueur >= R &&
                     lire_entete(fc, nblocs * 16u, h);
    if (!bon) {
        if (threadIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    const trc_disposition disp = disposition(dims, j);
    uint8_t* mat = emplacement + disp.base;
    uint32_t* codes = reinterpret_cast<uint32_t*>(mat);
    const uint8_t* ech = mat + disp.echelles;  // written by decoder_echelles
    const uint8_t* __restrict__ med = fm.p;

    const DemiVague dv = demi_vague();
    const uint32_t v = __lane_id() & 31u;
    const uint32_t vagues_bloc = blockDim.x >> 6;
    const uint32_t vague = blockIdx.x * vagues_bloc + (threadIdx.x >> 6);
    const uint32_t n_vagues = gridDim.x * vagues_bloc;
    const uint32_t nmacro = h.P / 128u;
    const uint32_t mots_utiles = nblocs * 4u;
    uint32_t hors_l = 0, pointeur = 0;
    for (uint32_t t0 = 2u * vague; t0 < h.T; t0 += 2u * n_vagues) {
        const uint32_t t = t0 + (dv.haut ? 1u : 0u);
        const bool tuile = t < h.T;
        const uint32_t nb_a = min(h.N, nmacro - t0 * h.N);
        const uint32_t nb = tuile ? min(h.N, nmacro - t * h.N) : 0u;
        uint32_t x = tuile ? h.etats[t * VOIES + v] : L;
        uint32_t ptr = tuile ? h.debut[t] : 0u;
        const uint32_t m0 = (tuile ? t : t0) * h.N;
        // word w = m*32 + v belongs to block w/4 = 8m + v/4; its context needs that block's scale
        // and its row median, fetched one macro-step ahead.
        uint32_t bloc = (m0 * VOIES + v) >> 2;
        uint32_t ligne = bloc / B, reste = bloc - ligne * B;
        bool valide = tuile && bloc < nblocs;
        uint32_t e_suiv = valide ? uint32_t(ech[bloc]) : 0u;
        uint32_t m_suiv = valide ? uint32_t(med[ligne]) : 0u;
        for (uint32_t m = 0; m < nb_a; ++m) {
            const bool actif = m < nb;
            const uint32_t ctx = valide ? classe_echelle(e_suiv, m_suiv) : 0u;
            const uint32_t w = (m0 + m) * VOIES + v;
            bloc += 8u;
            reste += 8u;
            while (reste >= B) {
                reste -= B;
                ++ligne;
            }
            valide = (m + 1u < nb) && bloc < nblocs;
            if (valide) {
                e_suiv = ech[bloc];
                m_suiv = med[ligne];
            }
            const uint32_t* lt = lut[ctx];
            uint32_t mot = 0;
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) mot |= pas_octet(x, ptr, lt, h.mots, h.W, dv, actif) << (8u * k);
            if (actif && w < mots_utiles) codes[w] = mot;
        }
        if (tuile) {
            hors_l += (x != L) ? 1u : 0u;
            const uint32_t attendu = (t + 1 < h.T) ? h.debut[t + 1] : h.W;
            pointeur += (v == 0 && ptr != attendu) ? 1u : 0u;
        }
    }
    verser_controle(controle, hors_l, pointeur);
}

struct DescDecodage {
    uint64_t partie, emplacement, luts, controle;
};
struct DescGemv {
    uint64_t matrice, x, y;
    uint32_t lignes, colonnes;
};

}  // namespace trc

extern "C" __global__ void __launch_bounds__(trc::FILS_ECHELLES)
decoder_echelles(const uint8_t* __restrict__ partie, uint8_t* __restrict__ emplacement,
                 const uint32_t* __restrict__ luts, trc_dims_expert dims, uint32_t* __restrict__ controle) {
    __shared__ uint32_t lut[trc::M];
    __shared__ uint8_t med[8192];
    trc::corps_echelles(partie, emplacement, luts, dims, controle, lut, med);
}

extern "C" __global__ void __launch_bounds__(trc::FILS_CODES)
decoder_codes(const uint8_t* __restrict__ partie, uint8_t* __restrict__ emplacement, const uint32_t* __restrict__ luts,
              trc_dims_expert dims, uint32_t* __restrict__ controle) {
    __shared__ uint32_t lut[3][trc::M];
    trc::corps_codes(partie, emplacement, luts, dims, controle, lut);
}

extern "C" __global__ void __launch_bounds__(trc::FILS_ECHELLES)
decoder_echelles_lot(const trc::DescDecodage* __restrict__ descs, trc_dims_expert dims) {
    __shared__ uint32_t lut[trc::M];
    __shared__ uint8_t med[8192];
    const trc::DescDecodage d = descs[blockIdx.z];
    trc::corps_echelles(reinterpret_cast<const uint8_t*>(d.partie), reinterpret_cast<uint8_t*>(d.emplacement),
                        reinterpret_cast<const uint32_t*>(d.luts), dims, reinterpret_cast<uint32_t*>(d.controle), lut,
                        med);
}

extern "C" __global__ void __launch_bounds__(trc::FILS_CODES)
decoder_codes_lot(const trc::DescDecodage* __restrict__ descs, trc_dims_expert dims) {
    __shared__ uint32_t lut[3][trc::M];
    const trc::DescDecodage d = descs[blockIdx.z];
    trc::corps_codes(reinterpret_cast<const uint8_t*>(d.partie), reinterpret_cast<uint8_t*>(d.emplacement),
                     reinterpret_cast<const uint32_t*>(d.luts), dims, reinterpret_cast<uint32_t*>(d.controle), lut);
}

// Raw-file path (flag bit 2): ECHELLES_BRUTES, CODES_BRUTS, BIAIS copied into the slot.
extern "C" __global__ void __launch_bounds__(trc::FILS_BRUT)
copier_brut(const uint8_t* __restrict__ partie, uint8_t* __restrict__ emplacement, trc_dims_expert dims,
            uint32_t* __restrict__ controle) {
    using namespace trc;
    const uint32_t j = blockIdx.y;
    const uint32_t R = choisir(dims.lignes, j), C = choisir(dims.colonnes, j);
    const uint32_t B = C / 32u, nblocs = R * B;
    DescFlux fe, fc, fb;
    const bool bon = (C % 32u == 0) && B > 0 && R > 0 && trouver_flux(partie, SORTE_ECHELLES_BRUTES, j, fe) &&
                     trouver_flux(partie, SORTE_CODES_BRUTS, j, fc) && trouver_flux(partie, SORTE_BIAIS, j, fb) &&
                     fe.produits == nblocs && fe.longueur >= nblocs && fc.produits == 16u * nblocs &&
                     fc.longueur >= 16u * nblocs && fb.produits == 4u * R && fb.longueur >= 4u * R;
    if (!bon) {
        if (threadIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    const trc_disposition disp = disposition(dims, j);
    uint8_t* mat = emplacement + disp.base;
    const uint32_t i0 = blockIdx.x * blockDim.x + threadIdx.x, pas = gridDim.x * blockDim.x;
    const uint4* cs = reinterpret_cast<const uint4*>(fc.p);
    uint4* cd = reinterpret_cast<uint4*>(mat);
    for (uint32_t i = i0; i < nblocs; i += pas) cd[i] = cs[i];
    for (uint32_t i = i0; i < nblocs; i += pas) mat[disp.echelles + i] = fe.p[i];
    const uint32_t* bs = reinterpret_cast<const uint32_t*>(fb.p);
    uint32_t* bd = reinterpret_cast<uint32_t*>(mat + disp.biais);
    for (uint32_t i = i0; i < R; i += pas) bd[i] = bs[i];
}

// ==================================================================================== GEMV MXFP4
namespace trc {

// Contribution of one block in the reference's fixed order (word t, byte k, low then high nibble).
__device__ __forceinline__ float produit_bloc(const uint4 q, const float4 (&xs)[8]) {
    const uint32_t mots[4] = {q.x, q.y, q.z, q.w};
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t w = mots[t];
        const float xa[4] = {xs[t].x, xs[t].y, xs[t].z, xs[t].w};
        const float xb[4] = {xs[4 + t].x, xs[4 + t].y, xs[4 + t].z, xs[4 + t].w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            s = fmaf(valeur_e2m1x2((w >> (8 * k)) & 15u), xa[k], s);
            s = fmaf(valeur_e2m1x2((w >> (8 * k + 4)) & 15u), xb[k], s);
        }
    }
    return s;
}

// Rows r0 .. r0+3 of one matrix, computed by one 32-lane half-wavefront exactly as one reference
// warp does: lane l takes blocks l, l+32, ...; 32-lane butterfly; lane 0 writes.
__device__ __forceinline__ void gemv_4_lignes(const uint8_t* __restrict__ mat, const float* __restrict__ x,
                                              float* __restrict__ y, uint32_t R, uint32_t C, uint32_t r0,
                                              uint32_t voie) {
    const uint32_t B = C / 32u;
    const trc_disposition d = disposition_matrice(R, C);
    const uint4* codes = reinterpret_cast<const uint4*>(mat);
    const uint8_t* ech = mat + d.echelles;
    const float* biais = reinterpret_cast<const float*>(mat + d.biais);
    const float4* x4 = reinterpret_cast<const float4*>(x);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t lig[4];
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) lig[i] = min(r0 + i, R - 1u);
    for (uint32_t b = voie; b < B; b += 32u) {
        float4 xs[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) xs[k] = x4[b * 8u + k];
        uint4 q[4];
        uint32_t e[4];
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const uint64_t beta = uint64_t(lig[i]) * B + b;
            q[i] = codes[beta];
            e[i] = ech[beta];
        }
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) acc[i] = fmaf(echelle_e8m0(e[i]), produit_bloc(q[i], xs), acc[i]);
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const float s = somme_demi_f32(acc[i]);
        if (voie == 0 && r0 + i < R) y[r0 + i] = s + biais[r0 + i];
    }
}

}  // namespace trc

extern "C" __global__ void __launch_bounds__(trc::GEMV_FILS)
gemv_mxfp4(const uint8_t* __restrict__ matrice, const float* __restrict__ x, float* __restrict__ y, uint32_t R,
           uint32_t C) {
    const uint32_t voie = threadIdx.x & 31u;
    const uint32_t r0 = (blockIdx.x * (trc::GEMV_FILS / 32u) + (threadIdx.x >> 5)) * 4u;
    if (r0 >= R || C % 32u != 0) return;
    trc::gemv_4_lignes(matrice, x, y, R, C, r0, voie);
}

extern "C" __global__ void __launch_bounds__(trc::GEMV_FILS) gemv_mxfp4_lot(const trc::DescGemv* __restrict__ descs) {
    const trc::DescGemv dsc = descs[blockIdx.y];
    const uint32_t voie = threadIdx.x & 31u;
    const uint32_t r0 = (blockIdx.x * (trc::GEMV_FILS / 32u) + (threadIdx.x >> 5)) * 4u;
    if (r0 >= dsc.lignes || dsc.colonnes % 32u != 0) return;
    trc::gemv_4_lignes(reinterpret_cast<const uint8_t*>(dsc.matrice), reinterpret_cast<const float*>(dsc.x),
                       reinterpret_cast<float*>(dsc.y), dsc.lignes, dsc.colonnes, r0, voie);
}

// =========================================================================== router, SwiGLU, combine

// y = W x (+ b), W f32 row-major: lane l of a half takes quads c = l, l+32, ...; butterfly
// (passe.cuh:104-130 order).
extern "C" __global__ void __launch_bounds__(trc::GEMV_FILS)
gemv_f32(const float* __restrict__ W, const float* __restrict__ x, const float* __restrict__ biais,
         float* __restrict__ y, uint32_t R, uint32_t C) {
    const uint32_t voie = threadIdx.x & 31u;
    const uint32_t r0 = (blockIdx.x * (trc::GEMV_FILS / 32u) + (threadIdx.x >> 5)) * 4u;
    if (r0 >= R || C % 4u != 0) return;
    const uint32_t C4 = C / 4u;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* W4 = reinterpret_cast<const float4*>(W);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t lig[4];
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) lig[i] = min(r0 + i, R - 1u);
    for (uint32_t c = voie; c < C4; c += 32u) {
        const float4 xv = x4[c];
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const float4 w = W4[uint64_t(lig[i]) * C4 + c];
            acc[i] = fmaf(w.x, xv.x, acc[i]);
            acc[i] = fmaf(w.y, xv.y, acc[i]);
            acc[i] = fmaf(w.z, xv.z, acc[i]);
            acc[i] = fmaf(w.w, xv.w, acc[i]);
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const float s = trc::somme_demi_f32(acc[i]);
        if (voie == 0 && r0 + i < R) y[r0 + i] = biais != nullptr ? s + biais[r0 + i] : s;
    }
}

// Top-k of E logits by (value desc, index asc); weights = softmax of the k in f64 (m = first,
// exp, ordered sum, division), rounded to f32. One wavefront: 64 lanes x 4 values (E <= 256).
extern "C" __global__ void __launch_bounds__(64)
routeur_topk(const float* __restrict__ logits, uint32_t E, uint32_t k, uint32_t* __restrict__ indices,
             float* __restrict__ poids, uint32_t* boite, uint32_t sequence) {
    using namespace trc;
    if (E == 0 || E > EXPERTS_MAX || k == 0 || k > TOPK_MAX || k > E) return;
    uint32_t choisi[TOPK_MAX];
    float w[TOPK_MAX];
    topk_vague(logits, E, k, choisi, w);
    if (threadIdx.x != 0) return;
#pragma unroll
    for (uint32_t r = 0; r < TOPK_MAX; ++r) {
        if (r < k) {
            indices[r] = choisi[r];
            poids[r] = w[r];
            if (boite != nullptr) {
                reinterpret_cast<volatile uint32_t*>(boite)[1 + r] = choisi[r];
                reinterpret_cast<volatile uint32_t*>(boite)[1 + k + r] = __float_as_uint(w[r]);
            }
        }
    }
    if (boite != nullptr) {
        __threadfence_system();
        reinterpret_cast<volatile uint32_t*>(boite)[0] = sequence;
    }
}

// The cache-biased router (passe.cuh:516-580): the k are chosen on the f32 score logit + biais
// (biais[e] = beta for an expert already in a VRAM slot, 0 else; score desc, index asc), then
// returned by unbiased logit desc, index asc, with the f64 softmax of the unbiased logits as
// weights. With a zero bias: routeur_topk's indices and weights, bit for bit. Same outputs and
// mailbox protocol as routeur_topk. A slot left unchosen (NaN scores) keeps index 0xFFFFFFFF and
// sorts last with weight 0.
extern "C" __global__ void __launch_bounds__(64)
routeur_topk_biais(const float* __restrict__ logits, const float* __restrict__ biais, uint32_t E, uint32_t k,
                   uint32_t* __restrict__ indices, float* __restrict__ poids, uint32_t* boite, uint32_t sequence) {
    using namespace trc;
    if (E == 0 || E > EXPERTS_MAX || k == 0 || k > TOPK_MAX || k > E) return;
    __shared__ float score[EXPERTS_MAX];
    for (uint32_t e = threadIdx.x; e < E; e += blockDim.x) score[e] = logits[e] + biais[e];
    __syncthreads();
    uint32_t choisi[TOPK_MAX];
    float w_score[TOPK_MAX];  // softmax of the scores: not used
    topk_vague(score, E, k, choisi, w_score);
    if (threadIdx.x != 0) return;
    float u[TOPK_MAX];
#pragma unroll
    for (uint32_t r = 0; r < TOPK_MAX; ++r) u[r] = r < k && choisi[r] < E ? logits[choisi[r]] : -INFINITY;
    for (uint32_t r = 1; r < k; ++r)
        for (uint32_t j = r; j > 0 && meilleur(u[j], choisi[j], u[j - 1], choisi[j - 1]); --j) {
            const float tv = u[j];
            u[j] = u[j - 1];
            u[j - 1] = tv;
            const uint32_t ti = choisi[j];
            choisi[j] = choisi[j - 1];
            choisi[j - 1] = ti;
        }
    double ex[TOPK_MAX];
    const double m = u[0];
    double z = 0.0;
    for (uint32_t r = 0; r < k; ++r) {
        ex[r] = exp(double(u[r]) - m);
        z += ex[r];
    }
    for (uint32_t r = 0; r < k; ++r) {
        const float w = float(ex[r] / z);
        indices[r] = choisi[r];
        poids[r] = w;
        if (boite != nullptr) {
            reinterpret_cast<volatile uint32_t*>(boite)[1 + r] = choisi[r];
            reinterpret_cast<volatile uint32_t*>(boite)[1 + k + r] = __float_as_uint(w);
        }
    }
    if (boite != nullptr) {
        __threadfence_system();
        reinterpret_cast<volatile uint32_t*>(boite)[0] = sequence;
    }
}

// gpt-oss clamped SwiGLU in f64, rounded once: g <- min(g,7); u <- clamp(u,-7,7);
// y = g / (1 + exp(-1.702 g)) * (u + 1).
extern "C" __global__ void __launch_bounds__(256)
swiglu_oai(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ y, uint32_t n) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= n) return;
    const double gv = fmin(double(g[i]), 7.0);
    const double uv = fmin(fmax(double(u[i]), -7.0), 7.0);
    y[i] = float(gv / (1.0 + exp(-1.702 * gv)) * (uv + 1.0));
}

// residu[i] += ((w0 s0[i] + w1 s1[i]) + w2 s2[i]) + ..., each product and sum rounded on its own.
extern "C" __global__ void __launch_bounds__(256)
combiner(float* __restrict__ residu, const float* __restrict__ sorties, uint32_t pas, const float* __restrict__ poids,
         uint32_t n, uint32_t d) {
#pragma clang fp contract(off)
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= d || n == 0) return;
    float s = poids != nullptr ? poids[0] * sorties[i] : sorties[i];
    for (uint32_t j = 1; j < n; ++j) {
        const float sj = sorties[uint64_t(j) * pas + i];
        const float p = poids != nullptr ? poids[j] * sj : sj;
        s = s + p;
    }
    residu[i] = residu[i] + s;
}

// ============================================================================ C-ABI launch layer
namespace {

using trc::usage;

inline hipStream_t flux_de(void* f) { return reinterpret_cast<hipStream_t>(f); }

int verifier_dims(const trc_dims_expert* dims) {
    if (dims == nullptr) return usage("dims absent");
    return trc_dims_verifier(dims);
}

}  // namespace

extern "C" int trc_decoder_expert(trc_vue partie, trc_vue emplacement, trc_vue luts, const trc_dims_expert* dims,
                                  trc_vue controle, void* flux) {
    int r = verifier_dims(dims);
    if (r != TRC_OK) return r;
    uint32_t g1[3], g2[3];
    trc_grilles_decodeur(dims, g1, g2);
    return trc_decoder_expert_grilles(partie, emplacement, luts, dims, controle, g1, g2, flux);
}

extern "C" int trc_decoder_expert_grilles(trc_vue partie, trc_vue emplacement, trc_vue luts,
                                          const trc_dims_expert* dims, trc_vue controle, const uint32_t g1[3],
                                          const uint32_t g2[3], void* flux) {
    int r = verifier_dims(dims);
    if (r != TRC_OK) return r;
    const uint64_t te = trc_taille_emplacement(dims);
    TRC_VERIFIER(partie.adresse != 0 && partie.octets >= 64, "partie de %llu o (en-tete de 64 o au moins)",
                 (unsigned long long)partie.octets);
    TRC_VERIFIER(partie.adresse % 16 == 0, "partie non alignee sur 16");
    TRC_VERIFIER(emplacement.octets >= te, "emplacement de %llu o, %llu o demandes",
                 (unsigned long long)emplacement.octets, (unsigned long long)te);
    TRC_VERIFIER(emplacement.adresse != 0 && emplacement.adresse % 256 == 0, "emplacement non aligne sur 256");
    TRC_VERIFIER(luts.adresse != 0 && luts.octets >= uint64_t(trc::LUTS_PAR_COUCHE) * 4, "LUT de %llu o",
                 (unsigned long long)luts.octets);
    TRC_VERIFIER(controle.adresse != 0 && controle.octets >= 16, "controle de moins de 16 o");
    TRC_VERIFIER(g1 != nullptr && g2 != nullptr && g1[1] == 3 && g2[1] == 3 && g1[0] > 0 && g2[0] > 0,
                 "grilles fausses");
    const hipStream_t f = flux_de(flux);
    auto p = reinterpret_cast<const uint8_t*>(partie.adresse);
    auto e = reinterpret_cast<uint8_t*>(emplacement.adresse);
    auto l = reinterpret_cast<const uint32_t*>(luts.adresse);
    auto c = reinterpret_cast<uint32_t*>(controle.adresse);
    hipLaunchKernelGGL(decoder_echelles, dim3(g1[0], 3, 1), dim3(trc::FILS_ECHELLES), 0, f, p, e, l, *dims, c);
    if ((r = trc::apres_lancement("decoder_echelles")) != TRC_OK) return r;
    hipLaunchKernelGGL(decoder_codes, dim3(g2[0], 3, 1), dim3(trc::FILS_CODES), 0, f, p, e, l, *dims, c);
    return trc::apres_lancement("decoder_codes");
}

extern "C" int trc_decoder_lot(trc_vue descs, uint32_t n, const trc_dims_expert* dims, void* flux) {
    int r = verifier_dims(dims);
    if (r != TRC_OK) return r;
    TRC_VERIFIER(n > 0 && n <= 65535, "lot de %u experts", n);
    TRC_VERIFIER(descs.adresse != 0 && descs.octets >= uint64_t(n) * sizeof(trc_desc_decodage),
                 "descripteurs trop courts");
    uint32_t g1[3], g2[3];
    trc_grilles_decodeur(dims, g1, g2);
    const hipStream_t f = flux_de(flux);
    auto d = reinterpret_cast<const trc::DescDecodage*>(descs.adresse);
    hipLaunchKernelGGL(decoder_echelles_lot, dim3(g1[0], 3, n), dim3(trc::FILS_ECHELLES), 0, f, d, *dims);
    if ((r = trc::apres_lancement("decoder_echelles_lot")) != TRC_OK) return r;
    hipLaunchKernelGGL(decoder_codes_lot, dim3(g2[0], 3, n), dim3(trc::FILS_CODES), 0, f, d, *dims);
    return trc::apres_lancement("decoder_codes_lot");
}

extern "C" int trc_copier_brut(trc_vue partie, trc_vue emplacement, const trc_dims_expert* dims, trc_vue controle,
                               void* flux) {
    int r = verifier_dims(dims);
    if (r != TRC_OK) return r;
    TRC_VERIFIER(partie.adresse != 0 && partie.octets >= 64, "partie trop courte");
    TRC_VERIFIER(partie.adresse % 16 == 0, "partie non alignee sur 16");
    TRC_VERIFIER(emplacement.adresse != 0 && emplacement.octets >= trc_taille_emplacement(dims),
                 "emplacement trop court");
    TRC_VERIFIER(emplacement.adresse % 256 == 0, "emplacement non aligne sur 256");
    TRC_VERIFIER(controle.adresse != 0 && controle.octets >= 16, "controle de moins de 16 o");
    uint32_t g[3];
    trc_grille_brut(dims, g);
    hipLaunchKernelGGL(copier_brut, dim3(g[0], 3, 1), dim3(trc::FILS_BRUT), 0, flux_de(flux),
                       reinterpret_cast<const uint8_t*>(partie.adresse), reinterpret_cast<uint8_t*>(emplacement.adresse),
                       *dims, reinterpret_cast<uint32_t*>(controle.adresse));
    return trc::apres_lancement("copier_brut");
}

extern "C" int trc_gemv(trc_vue matrice, trc_vue x, trc_vue y, uint32_t lignes, uint32_t colonnes, void* flux) {
    TRC_VERIFIER(lignes > 0 && colonnes > 0 && colonnes % 32 == 0, "forme %u x %u", lignes, colonnes);
    const uint64_t pas = trc::disposition_matrice(lignes, colonnes).pas;
    TRC_VERIFIER(matrice.adresse != 0 && matrice.octets >= pas, "matrice de %llu o, %llu o demandes",
                 (unsigned long long)matrice.octets, (unsigned long long)pas);
    TRC_VERIFIER(matrice.adresse % 256 == 0, "matrice non alignee sur 256");
    TRC_VERIFIER(x.adresse != 0 && x.octets >= 4ull * colonnes && x.adresse % 16 == 0,
                 "x trop court ou non aligne sur 16");
    TRC_VERIFIER(y.adresse != 0 && y.octets >= 4ull * lignes, "y trop court");
    hipLaunchKernelGGL(gemv_mxfp4, dim3((lignes + trc::GEMV_LIGNES_PAR_BLOC - 1) / trc::GEMV_LIGNES_PAR_BLOC),
                       dim3(trc::GEMV_FILS), 0, flux_de(flux), reinterpret_cast<const uint8_t*>(matrice.adresse),
                       reinterpret_cast<const float*>(x.adresse), reinterpret_cast<float*>(y.adresse), lignes,
                       colonnes);
    return trc::apres_lancement("gemv_mxfp4");
}

extern "C" int trc_gemv_lot(trc_vue descs, uint32_t n, uint32_t lignes_max, void* flux) {
    TRC_VERIFIER(n > 0 && n <= 65535, "lot de %u produits", n);
    TRC_VERIFIER(descs.adresse != 0 && descs.octets >= uint64_t(n) * sizeof(trc_desc_gemv), "descripteurs trop courts");
    TRC_VERIFIER(lignes_max > 0, "lignes_max nul");
    hipLaunchKernelGGL(gemv_mxfp4_lot,
                       dim3((lignes_max + trc::GEMV_LIGNES_PAR_BLOC - 1) / trc::GEMV_LIGNES_PAR_BLOC, n),
                       dim3(trc::GEMV_FILS), 0, flux_de(flux), reinterpret_cast<const trc::DescGemv*>(descs.adresse));
    return trc::apres_lancement("gemv_mxfp4_lot");
}

extern "C" int trc_gemv_f32(trc_vue w, trc_vue x, trc_vue biais, trc_vue y, uint32_t lignes, uint32_t colonnes,
                            void* flux) {
    TRC_VERIFIER(lignes > 0 && colonnes > 0 && colonnes % 4 == 0, "forme %u x %u", lignes, colonnes);
    TRC_VERIFIER(w.adresse != 0 && w.octets >= 4ull * lignes * colonnes && w.adresse % 16 == 0,
                 "matrice f32 trop courte ou non alignee sur 16");
    TRC_VERIFIER(x.adresse != 0 && x.octets >= 4ull * colonnes && x.adresse % 16 == 0,
                 "x trop court ou non aligne sur 16");
    TRC_VERIFIER(y.adresse != 0 && y.octets >= 4ull * lignes, "y trop court");
    TRC_VERIFIER(biais.adresse == 0 || biais.octets >= 4ull * lignes, "biais trop court");
    hipLaunchKernelGGL(gemv_f32, dim3((lignes + trc::GEMV_LIGNES_PAR_BLOC - 1) / trc::GEMV_LIGNES_PAR_BLOC),
                       dim3(trc::GEMV_FILS), 0, flux_de(flux), reinterpret_cast<const float*>(w.adresse),
                       reinterpret_cast<const float*>(x.adresse), reinterpret_cast<const float*>(biais.adresse),
                       reinterpret_cast<float*>(y.adresse), lignes, colonnes);
    return trc::apres_lancement("gemv_f32");
}

extern "C" int trc_routeur_topk(trc_vue logits, uint32_t experts, uint32_t k, trc_vue indices, trc_vue poids,
                                uint64_t boite, uint32_t sequence, void* flux) {
    TRC_VERIFIER(experts > 0 && experts <= 256 && k > 0 && k <= 8 && k <= experts, "top-%u sur %u", k, experts);
    TRC_VERIFIER(logits.adresse != 0 && logits.octets >= 4ull * experts && indices.adresse != 0 &&
                     indices.octets >= 4ull * k && poids.adresse != 0 && poids.octets >= 4ull * k,
                 "routeur : vues trop courtes");
    hipLaunchKernelGGL(routeur_topk, dim3(1), dim3(64), 0, flux_de(flux), reinterpret_cast<const float*>(logits.adresse),
                       experts, k, reinterpret_cast<uint32_t*>(indices.adresse), reinterpret_cast<float*>(poids.adresse),
                       reinterpret_cast<uint32_t*>(boite), sequence);
    return trc::apres_lancement("routeur_topk");
}

extern "C" int trc_routeur_topk_biais(trc_vue logits, trc_vue biais, uint32_t experts, uint32_t k, trc_vue indices,
                                      trc_vue poids, uint64_t boite, uint32_t sequence, void* flux) {
    TRC_VERIFIER(experts > 0 && experts <= 256 && k > 0 && k <= 8 && k <= experts, "top-%u sur %u", k, experts);
    TRC_VERIFIER(logits.adresse != 0 && logits.octets >= 4ull * experts && biais.adresse != 0 &&
                     biais.octets >= 4ull * experts && indices.adresse != 0 && indices.octets >= 4ull * k &&
                     poids.adresse != 0 && poids.octets >= 4ull * k,
                 "routeur biaise : vues trop courtes");
    hipLaunchKernelGGL(routeur_topk_biais, dim3(1), dim3(64), 0, flux_de(flux),
                       reinterpret_cast<const float*>(logits.adresse), reinterpret_cast<const float*>(biais.adresse),
                       experts, k, reinterpret_cast<uint32_t*>(indices.adresse), reinterpret_cast<float*>(poids.adresse),
                       reinterpret_cast<uint32_t*>(boite), sequence);
    return trc::apres_lancement("routeur_topk_biais");
}

extern "C" int trc_swiglu_oai(trc_vue g, trc_vue u, trc_vue y, uint32_t n, void* flux) {
    const uint64_t o = 4ull * n;
    TRC_VERIFIER(n > 0 && g.adresse && u.adresse && y.adresse && g.octets >= o && u.octets >= o && y.octets >= o,
                 "swiglu : vues trop courtes");
    hipLaunchKernelGGL(swiglu_oai, dim3((n + 255) / 256), dim3(256), 0, flux_de(flux),
                       reinterpret_cast<const float*>(g.adresse), reinterpret_cast<const float*>(u.adresse),
                       reinterpret_cast<float*>(y.adresse), n);
    return trc::apres_lancement("swiglu_oai");
}

extern "C" int trc_combiner(trc_vue residu, trc_vue sorties, uint32_t pas, trc_vue poids, uint32_t n, uint32_t d,
                            void* flux) {
    TRC_VERIFIER(n > 0 && d > 0 && (n == 1 || pas >= d), "combiner %u sorties de %u (pas %u)", n, d, pas);
    TRC_VERIFIER(residu.adresse && sorties.adresse && residu.octets >= 4ull * d &&
                     sorties.octets >= 4ull * ((uint64_t(n) - 1) * pas + d),
                 "combiner : vues trop courtes");
    TRC_VERIFIER(poids.adresse == 0 || poids.octets >= 4ull * n, "poids trop courts");
    hipLaunchKernelGGL(combiner, dim3((d + 255) / 256), dim3(256), 0, flux_de(flux),
                       reinterpret_cast<float*>(residu.adresse), reinterpret_cast<const float*>(sorties.adresse), pas,
                       reinterpret_cast<const float*>(poids.adresse), n, d);
    return trc::apres_lancement("combiner");
}
