// fusion.hip — the fused expert path for gfx950: rANS decoding of the .trc v1.2 streams feeds the
// MXFP4 dequant and the GEMV directly; decoded code bytes live only in registers and are never
// written to HBM. Built from four kernels chained on one stream:
//
//   fusion_echelles  DELTA tiles -> E8M0 scales of the selected matrices (a small workspace);
//   fusion_gemv      CODES_CTX tiles -> per-(row, tile) partial sums of y = W x, decoded bytes
//                    dequantised and multiplied in registers;
//   fusion_finir     y[r] = fixed-order sum of the row's tile partials + bias;
//   fusion_routeur / fusion_taches  (MoE layer) router logits, then the job table of the
//                    selected experts, built on the device from the top-k indices.
//
// Mapping: one wavefront = two rANS tiles (lanes 0-31, 32-63). In a macro-step, lane v of a tile
// produces the 4 code bytes 4(v%4) .. 4(v%4)+3 of block 8m + v/4, i.e. the weights of columns
// 32b + 4(v%4) + k (low nibbles) and 32b + 16 + 4(v%4) + k (high nibbles): two float4 of x. Each
// lane accumulates its block contributions per row; rows are closed by a 32-lane reduction when
// the tile's first block enters a new row (a row has >= 8 blocks, so one macro-step touches at
// most two rows). Every (row, tile) partial is written exactly once and summed in tile order by
// the finisher: results are deterministic, without floating-point atomics.
#include <hip/hip_runtime.h>

#include "chrono.hpp"
#include "commun.hpp"
#include "erreurs.hpp"

// Reference-API kernels (noyaux.hip) reused by the MoE layer.
extern "C" __global__ void routeur_topk(const float* logits, uint32_t E, uint32_t k, uint32_t* indices, float* poids,
                                       uint32_t* boite, uint32_t sequence);
extern "C" __global__ void combiner(float* residu, const float* sorties, uint32_t pas, const float* poids, uint32_t n,
                                    uint32_t d);

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

__device__ __forceinline__ uint32_t premiere_tuile(uint32_t ligne, uint32_t B, uint32_t blocs_par_tuile) {
    return (ligne * B) / blocs_par_tuile;
}

// ----------------------------------------------------------------------- DELTA -> scales only
__device__ __forceinline__ void corps_echelles_fusion(const Tache& tc, const uint32_t* lut, uint8_t* med_lds,
                                                      uint32_t* __restrict__ controle) {
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
        for (uint32_t i = threadIdx.x; i < R; i += blockDim.x) med_lds[i] = fm.p[i];
        med = med_lds;
    }
    __syncthreads();
    uint8_t* ech = reinterpret_cast<uint8_t*>(tc.ech);
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

// ------------------------------------------------------------ CODES_CTX -> partial sums of W x
__device__ __forceinline__ void corps_gemv_fusion(const Tache& tc, const uint32_t (*lut)[M],
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
    const uint8_t* __restrict__ med = fm.p;
    const uint8_t* __restrict__ ech = reinterpret_cast<const uint8_t*>(tc.ech);
    const float4* __restrict__ x4 = reinterpret_cast<const float4*>(tc.x);
    float* __restrict__ partiels = reinterpret_cast<float*>(tc.partiels);
    const uint32_t kmax = tc.kmax;
    const uint32_t bpt = 8u * h.N;  // blocks per tile

    const DemiVague dv = demi_vague();
    const uint32_t v = __lane_id() & 31u;
    const uint32_t q = v >> 2, q4 = v & 3u;
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
        const uint32_t m0 = (tuile ? t : t0) * h.N;
        uint32_t bloc = m0 * 8u + q;
        uint32_t ligne = bloc / B, b = bloc - ligne * B;
        uint32_t rho = (m0 * 8u) / B, base_b = m0 * 8u - rho * B;  // row of the tile's first block
        bool valide = tuile && bloc < nblocs;
        uint32_t e_suiv = valide ? uint32_t(ech[bloc]) : 0u;
        uint32_t m_suiv = valide ? uint32_t(med[ligne]) : 0u;
        float acc_a = 0.0f, acc_b = 0.0f;
        for (uint32_t m = 0; m < nb_a; ++m) {
            const bool actif = m < nb;
            const bool bloc_ok = valide;
            const uint32_t e_cur = e_suiv;
            const uint32_t ctx = bloc_ok ? classe_echelle(e_suiv, m_suiv) : 0u;
            const uint32_t b_cur = b, ligne_cur = ligne;
            bloc += 8u;
            b += 8u;
            while (b >= B) {
                b -= B;
                ++ligne;
            }
            valide = (m + 1u < nb) && bloc < nblocs;
            if (valide) {
                e_suiv = ech[bloc];
                m_suiv = med[ligne];
            }
            float4 xa = make_float4(0.f, 0.f, 0.f, 0.f), xb = xa;
            if (bloc_ok) {
                xa = x4[8u * b_cur + q4];
                xb = x4[8u * b_cur + 4u + q4];
            }
            const uint32_t* lt = lut[ctx];
            uint32_t mot = 0;
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) mot |= pas_octet(x, ptr, lt, h.mots, h.W, dv, actif) << (8u * k);
            if (actif && bloc_ok) {
                float d = 0.0f;
                d = fmaf(valeur_e2m1x2(mot & 15u), xa.x, d);
                d = fmaf(valeur_e2m1x2((mot >> 4) & 15u), xb.x, d);
                d = fmaf(valeur_e2m1x2((mot >> 8) & 15u), xa.y, d);
                d = fmaf(valeur_e2m1x2((mot >> 12) & 15u), xb.y, d);
                d = fmaf(valeur_e2m1x2((mot >> 16) & 15u), xa.z, d);
                d = fmaf(valeur_e2m1x2((mot >> 20) & 15u), xb.z, d);
                d = fmaf(valeur_e2m1x2((mot >> 24) & 15u), xa.w, d);
                d = fmaf(valeur_e2m1x2(mot >> 28), xb.w, d);
                const float c = d * echelle_e8m0(e_cur);
                if (ligne_cur == rho)
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
            if (__ballot(avance) != 0) {
                const float s = somme_demi_f32(acc_a);
                if (avance) {
                    if (v == 0 && rho < R) partiels[rho * kmax + (t - premiere_tuile(rho, B, bpt))] = s;
                    acc_a = acc_b;
                    acc_b = 0.0f;
                    ++rho;
                }
            }
        }
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
            pointeur += (v == 0 && ptr != attendu) ? 1u : 0u;
        }
    }
    verser_controle(controle, hors_l, pointeur);
}

}  // namespace trc

// The job of block (x, y) is taches[y]; the layer's LUTs u32[3][4][4096] are shared by all jobs.
extern "C" __global__ void __launch_bounds__(128)
fusion_echelles(const trc::Tache* __restrict__ taches, const uint32_t* __restrict__ luts,
                uint32_t* __restrict__ controle) {
    __shared__ uint32_t lut[trc::M];
    __shared__ uint8_t med[8192];
    const trc::Tache tc = taches[blockIdx.y];
    const uint32_t* src = luts + (uint64_t(tc.j) * 4u + 0u) * trc::M;
    for (uint32_t i = threadIdx.x; i < trc::M; i += blockDim.x) lut[i] = src[i];
    __syncthreads();
    trc::corps_echelles_fusion(tc, lut, med, controle);
}

extern "C" __global__ void __launch_bounds__(256)
fusion_gemv(const trc::Tache* __restrict__ taches, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    __shared__ uint32_t lut[3][trc::M];
    const trc::Tache tc = taches[blockIdx.y];
    const uint32_t* src = luts + (uint64_t(tc.j) * 4u + 1u) * trc::M;
    uint32_t* dst = &lut[0][0];
    for (uint32_t i = threadIdx.x; i < 3u * trc::M; i += blockDim.x) dst[i] = src[i];
    __syncthreads();
    trc::corps_gemv_fusion(tc, lut, controle);
}

// sorties[y * pas + r] = fixed-order sum of the partials of row r + bias[r], for job y.
extern "C" __global__ void __launch_bounds__(256)
fusion_finir(const trc::Tache* __restrict__ taches, float* __restrict__ sorties, uint32_t pas) {
    using namespace trc;
    const Tache tc = taches[blockIdx.y];
    const uint32_t r = blockIdx.x * 256u + threadIdx.x;
    if (r >= tc.lignes) return;
    const uint8_t* partie = reinterpret_cast<const uint8_t*>(tc.partie);
    const uint32_t B = tc.colonnes / 32u;
    DescFlux fc, fb;
    EnteteRans h;
    if (!(trouver_flux(partie, SORTE_CODES_CTX, tc.j, fc) && trouver_flux(partie, SORTE_BIAIS, tc.j, fb) &&
          fb.longueur >= 4u * tc.lignes && lire_entete(fc, tc.lignes * B * 16u, h) && B >= 8u &&
          (B - 1u) / (8u * h.N) + 2u <= tc.kmax))
        return;  // counted by fusion_gemv
    const uint32_t bpt = 8u * h.N;
    const uint32_t t0 = (r * B) / bpt, t1 = (r * B + B - 1u) / bpt;
    const float* p = reinterpret_cast<const float*>(tc.partiels) + uint64_t(r) * tc.kmax;
    float s = p[0];
    for (uint32_t k = 1; k <= t1 - t0; ++k) s += p[k];
    sorties[uint64_t(blockIdx.y) * pas + r] = s + reinterpret_cast<const float*>(fb.p)[r];
}

// Router logits: y = W x (+ b) with W bf16 row-major (E x C), in the reference gemv_f32 order
// (bf16 -> f32 is exact, so the bits equal gemv_f32 on the widened matrix).
extern "C" __global__ void __launch_bounds__(256)
fusion_routeur(const uint16_t* __restrict__ W, const float* __restrict__ x, const float* __restrict__ biais,
               float* __restrict__ y, uint32_t R, uint32_t C) {
    const uint32_t voie = threadIdx.x & 31u;
    const uint32_t r0 = (blockIdx.x * 8u + (threadIdx.x >> 5)) * 4u;
    if (r0 >= R) return;
    const uint32_t C4 = C / 4u;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const uint2* W4 = reinterpret_cast<const uint2*>(W);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t lig[4];
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) lig[i] = min(r0 + i, R - 1u);
    for (uint32_t c = voie; c < C4; c += 32u) {
        const float4 xv = x4[c];
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const uint2 w = W4[uint64_t(lig[i]) * C4 + c];
            acc[i] = fmaf(__uint_as_float(w.x << 16), xv.x, acc[i]);
            acc[i] = fmaf(__uint_as_float(w.x & 0xFFFF0000u), xv.y, acc[i]);
            acc[i] = fmaf(__uint_as_float(w.y << 16), xv.z, acc[i]);
            acc[i] = fmaf(__uint_as_float(w.y & 0xFFFF0000u), xv.w, acc[i]);
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const float s = trc::somme_demi_f32(acc[i]);
        if (voie == 0 && r0 + i < R) y[r0 + i] = biais != nullptr ? s + biais[r0 + i] : s;
    }
}

// Job tables of a MoE layer from the top-k indices: for selected expert i, jobs 2i (gate) and
// 2i+1 (up) in table `gu` against x, job i (down) in table `bas` against act + i*lignes, and the
// DELTA jobs (3 per expert) in `delta`. Workspace pieces are laid out per (i, j).
namespace trc {
struct ParamsTaches {
    uint64_t parties;   // u64[E] part addresses
    uint64_t indices;   // u32[k]
    uint64_t x;         // f32[C]
    uint64_t act;       // f32[k * R]
    uint64_t ech;       // scales: (i*3 + j) * pas_ech
    uint64_t partiels;  // partials: (i*3 + j) * pas_partiels
    uint64_t delta, gu, bas;  // Tache tables
    uint64_t pas;             // workspace bytes per (i, j)
    uint32_t lignes[3], colonnes[3], kmax[3];
    uint32_t k, E;
};
}  // namespace trc

extern "C" __global__ void __launch_bounds__(64) fusion_taches(trc::ParamsTaches p, uint32_t* __restrict__ controle) {
    using namespace trc;
    const uint32_t i = threadIdx.x;
    if (i >= p.k) return;
    const uint32_t e = reinterpret_cast<const uint32_t*>(p.indices)[i];
    uint64_t partie = 0;
    if (e < p.E) {
        partie = reinterpret_cast<const uint64_t*>(p.parties)[e];
    } else {
        atomicAdd(&controle[CTL_FORMAT], 1u);
    }
    Tache* td = reinterpret_cast<Tache*>(p.delta);
    Tache* tgu = reinterpret_cast<Tache*>(p.gu);
    Tache* tb = reinterpret_cast<Tache*>(p.bas);
    for (uint32_t j = 0; j < 3; ++j) {
        Tache t;
        t.partie = partie;
        t.j = j;
        t.kmax = p.kmax[j];
        t.lignes = p.lignes[j];
        t.colonnes = p.colonnes[j];
        t.ech = p.ech + uint64_t(i * 3 + j) * p.pas;
        t.partiels = p.partiels + uint64_t(i * 3 + j) * p.pas;
        t.x = j < 2 ? p.x : p.act + uint64_t(i) * p.colonnes[2] * 4u;
        td[i * 3 + j] = t;
        if (j < 2)
            tgu[i * 2 + j] = t;
        else
            tb[i] = t;
    }
}

// act[i*R + r] = swiglu(gu[2i*R + r], gu[(2i+1)*R + r]) for the k experts (gpt-oss clamped SwiGLU,
// f64, one rounding — the reference swiglu_oai).
extern "C" __global__ void __launch_bounds__(256)
fusion_swiglu(const float* __restrict__ gu, float* __restrict__ act, uint32_t R, uint32_t k) {
    const uint32_t r = blockIdx.x * 256u + threadIdx.x, i = blockIdx.y;
    if (r >= R || i >= k) return;
    const double gv = fmin(double(gu[uint64_t(2 * i) * R + r]), 7.0);
    const double uv = fmin(fmax(double(gu[uint64_t(2 * i + 1) * R + r]), -7.0), 7.0);
    act[uint64_t(i) * R + r] = float(gv / (1.0 + exp(-1.702 * gv)) * (uv + 1.0));
}

// ============================================================================ C-ABI launch layer
namespace {

using trc::usage;
using trc::Tache;

inline hipStream_t flux_de(void* f) { return reinterpret_cast<hipStream_t>(f); }

uint32_t kmax_pour(uint32_t colonnes, uint32_t n_codes) {
    const uint32_t B = colonnes / 32u;
    return (B - 1u) / (8u * n_codes) + 2u;
}

uint64_t al(uint64_t x) { return (x + 255u) & ~uint64_t(255); }

uint32_t grille_tuiles(uint64_t octets, uint32_t N, uint32_t tuiles_par_bloc) {
    const uint64_t macro = (octets + 127) / 128;
    const uint64_t T = (macro + N - 1) / N;
    const uint64_t g = (T + tuiles_par_bloc - 1) / tuiles_par_bloc;
    return uint32_t(g < 1 ? 1 : g);
}

// Workspace of one matrix job: scales then partial sums.
uint64_t pas_tache(uint32_t R, uint32_t C, uint32_t n_codes) {
    return al(uint64_t(R) * (C / 32)) + al(4ull * R * kmax_pour(C, n_codes));
}

int verifier_forme(const trc_dims_expert* dims, uint32_t n_codes) {
    if (dims == nullptr) return usage("dims absent");
    int r = trc_dims_verifier(dims);
    if (r != TRC_OK) return r;
    for (int j = 0; j < 3; ++j)
        if (dims->colonnes[j] / 32 < 8) return usage("matrice %d : moins de 8 blocs par ligne (chemin fusionne)", j);
    if (n_codes == 0 || n_codes > 65535) return usage("N de CODES_CTX %u", n_codes);
    return TRC_OK;
}

int lancer_chaine(const Tache* taches_dev, uint32_t n, const uint32_t* luts, uint32_t* ctl, uint32_t R, uint32_t C,
                  uint32_t n_delta, uint32_t n_codes, bool echelles, hipStream_t f) {
    const uint32_t B = C / 32;
    if (echelles)
        TRC_LANCER(fusion_echelles, dim3(grille_tuiles(uint64_t(R) * B, n_delta, 4), n), dim3(128), f, taches_dev, luts,
                   ctl);
    TRC_LANCER(fusion_gemv, dim3(grille_tuiles(16ull * R * B, n_codes, 8), n), dim3(256), f, taches_dev, luts, ctl);
    return TRC_OK;
}

}  // namespace

extern "C" uint64_t trc_taille_travail_gemv_fusionnee(uint32_t lignes, uint32_t colonnes, uint32_t n_codes) {
    if (colonnes / 32 < 8 || n_codes == 0) return 0;
    return al(sizeof(Tache)) + pas_tache(lignes, colonnes, n_codes);
}

// Config 1: one matrix j of a part, y = W_j x + b_j, decoded in registers.
extern "C" int trc_gemv_fusionnee(trc_vue partie, uint32_t j, trc_vue luts, uint32_t lignes, uint32_t colonnes,
                                  trc_vue x, trc_vue y, trc_vue controle, trc_vue travail, uint32_t n_delta,
                                  uint32_t n_codes, void* flux) {
    TRC_VERIFIER(j < 3, "matrice %u", j);
    TRC_VERIFIER(lignes > 0 && colonnes % 32 == 0 && colonnes / 32 >= 8, "forme %u x %u", lignes, colonnes);
    TRC_VERIFIER(n_delta > 0 && n_codes > 0 && n_delta <= 65535 && n_codes <= 65535, "N faux");
    TRC_VERIFIER(partie.adresse && partie.octets >= 64, "partie trop courte");
    TRC_VERIFIER(luts.adresse && luts.octets >= uint64_t(trc::LUTS_PAR_COUCHE) * 4, "LUT trop courtes");
    TRC_VERIFIER(x.adresse && x.octets >= 4ull * colonnes && x.adresse % 16 == 0, "x trop court ou non aligne");
    TRC_VERIFIER(y.adresse && y.octets >= 4ull * lignes, "y trop court");
    TRC_VERIFIER(controle.adresse && controle.octets >= 16, "controle de moins de 16 o");
    const uint64_t besoin = trc_taille_travail_gemv_fusionnee(lignes, colonnes, n_codes);
    TRC_VERIFIER(travail.adresse && travail.octets >= besoin && travail.adresse % 256 == 0,
                 "travail de %llu o, %llu o demandes (aligne sur 256)", (unsigned long long)travail.octets,
                 (unsigned long long)besoin);
    Tache t;
    t.partie = partie.adresse;
    t.x = x.adresse;
    t.ech = travail.adresse + al(sizeof(Tache));
    t.partiels = t.ech + al(uint64_t(lignes) * (colonnes / 32));
    t.j = j;
    t.kmax = kmax_pour(colonnes, n_codes);
    t.lignes = lignes;
    t.colonnes = colonnes;
    const hipStream_t f = flux_de(flux);
    hipError_t e = hipMemcpyAsync(reinterpret_cast<void*>(travail.adresse), &t, sizeof(t), hipMemcpyHostToDevice, f);
    if (e != hipSuccess) return trc::erreur_hip("hipMemcpyAsync", e);
    const Tache* td = reinterpret_cast<const Tache*>(travail.adresse);
    auto ctl = reinterpret_cast<uint32_t*>(controle.adresse);
    int r = lancer_chaine(td, 1, reinterpret_cast<const uint32_t*>(luts.adresse), ctl, lignes, colonnes, n_delta,
                          n_codes, true, f);
    if (r != TRC_OK) return r;
    TRC_LANCER(fusion_finir, dim3((lignes + 255) / 256, 1), dim3(256), f, td, reinterpret_cast<float*>(y.adresse), 0u);
    return TRC_OK;
}

extern "C" uint64_t trc_taille_travail_expert_fusionne(const trc_dims_expert* dims, uint32_t n_codes) {
    if (verifier_forme(dims, n_codes) != TRC_OK) return 0;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0];
    return al(3 * sizeof(Tache)) + 3 * pas_tache(dims->lignes[2] > R ? dims->lignes[2] : R,
                                                 dims->colonnes[2] > C ? dims->colonnes[2] : C, n_codes) +
           al(4ull * 2 * R) + al(4ull * R);
}

// Config 2: one expert, s = W_down swiglu(W_gate x + b_gate, W_up x + b_up) + b_down, every matrix
// decoded in registers (gate/up/down = matrices 0/1/2 of the part).
extern "C" int trc_expert_fusionne(trc_vue partie, trc_vue luts, const trc_dims_expert* dims, trc_vue x,
                                   trc_vue sortie, trc_vue controle, trc_vue travail, uint32_t n_delta,
                                   uint32_t n_codes, void* flux) {
    int r = verifier_forme(dims, n_codes);
    if (r != TRC_OK) return r;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0];
    TRC_VERIFIER(dims->lignes[1] == R && dims->colonnes[1] == C && dims->colonnes[2] == R,
                 "gate, up et down incompatibles (down doit lire les %u sorties de la SwiGLU)", R);
    TRC_VERIFIER(n_delta > 0 && n_delta <= 65535, "N de DELTA %u", n_delta);
    TRC_VERIFIER(partie.adresse && partie.octets >= 64, "partie trop courte");
    TRC_VERIFIER(luts.adresse && luts.octets >= uint64_t(trc::LUTS_PAR_COUCHE) * 4, "LUT trop courtes");
    TRC_VERIFIER(x.adresse && x.octets >= 4ull * C && x.adresse % 16 == 0, "x trop court ou non aligne");
    TRC_VERIFIER(sortie.adresse && sortie.octets >= 4ull * dims->lignes[2], "sortie trop courte");
    TRC_VERIFIER(controle.adresse && controle.octets >= 16, "controle de moins de 16 o");
    const uint64_t besoin = trc_taille_travail_expert_fusionne(dims, n_codes);
    TRC_VERIFIER(travail.adresse && travail.octets >= besoin && travail.adresse % 256 == 0,
                 "travail de %llu o, %llu o demandes (aligne sur 256)", (unsigned long long)travail.octets,
                 (unsigned long long)besoin);
    const uint32_t Rm = dims->lignes[2] > R ? dims->lignes[2] : R;
    const uint32_t Cm = dims->colonnes[2] > C ? dims->colonnes[2] : C;
    const uint64_t pas = pas_tache(Rm, Cm, n_codes);
    const uint64_t base = travail.adresse + al(3 * sizeof(Tache));
    const uint64_t gu = base + 3 * pas, act = gu + al(4ull * 2 * R);
    Tache t[3];
    for (uint32_t j = 0; j < 3; ++j) {
        t[j].partie = partie.adresse;
        t[j].j = j;
        t[j].lignes = dims->lignes[j];
        t[j].colonnes = dims->colonnes[j];
        t[j].kmax = kmax_pour(dims->colonnes[j], n_codes);
        t[j].ech = base + j * pas;
        t[j].partiels = t[j].ech + al(uint64_t(Rm) * (Cm / 32));
        t[j].x = j < 2 ? x.adresse : act;
    }
    const hipStream_t f = flux_de(flux);
    hipError_t e = hipMemcpyAsync(reinterpret_cast<void*>(travail.adresse), t, sizeof(t), hipMemcpyHostToDevice, f);
    if (e != hipSuccess) return trc::erreur_hip("hipMemcpyAsync", e);
    const Tache* td = reinterpret_cast<const Tache*>(travail.adresse);
    const uint32_t* l = reinterpret_cast<const uint32_t*>(luts.adresse);
    auto ctl = reinterpret_cast<uint32_t*>(controle.adresse);
    const uint32_t B = C / 32;
    TRC_LANCER(fusion_echelles, dim3(grille_tuiles(uint64_t(Rm) * (Cm / 32), n_delta, 4), 3), dim3(128), f, td, l, ctl);
    TRC_LANCER(fusion_gemv, dim3(grille_tuiles(16ull * R * B, n_codes, 8), 2), dim3(256), f, td, l, ctl);
    TRC_LANCER(fusion_finir, dim3((R + 255) / 256, 2), dim3(256), f, td, reinterpret_cast<float*>(gu), R);
    TRC_LANCER(fusion_swiglu, dim3((R + 255) / 256, 1), dim3(256), f, reinterpret_cast<const float*>(gu),
               reinterpret_cast<float*>(act), R, 1u);
    const uint32_t R2 = dims->lignes[2], B2 = dims->colonnes[2] / 32;
    TRC_LANCER(fusion_gemv, dim3(grille_tuiles(16ull * R2 * B2, n_codes, 8), 1), dim3(256), f, td + 2, l, ctl);
    TRC_LANCER(fusion_finir, dim3((R2 + 255) / 256, 1), dim3(256), f, td + 2, reinterpret_cast<float*>(sortie.adresse),
               0u);
    return TRC_OK;
}

extern "C" uint64_t trc_taille_travail_couche_moe(const trc_dims_expert* dims, uint32_t experts, uint32_t k,
                                                  uint32_t n_codes) {
    if (verifier_forme(dims, n_codes) != TRC_OK || k == 0 || k > 8 || experts == 0) return 0;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0];
    const uint32_t Rm = dims->lignes[2] > R ? dims->lignes[2] : R;
    const uint32_t Cm = dims->colonnes[2] > C ? dims->colonnes[2] : C;
    return al(3ull * k * sizeof(Tache)) * 2 + al(4ull * experts) + 3ull * k * pas_tache(Rm, Cm, n_codes) +
           al(4ull * 2 * k * R) + al(4ull * k * R) + al(4ull * k * dims->lignes[2]);
}

// Config 3: one MoE layer decode step at batch 1. logits = W_r x (+ b_r) (W_r bf16, experts x C),
// top-k with softmax weights (indices/poids written out), then for the k selected experts the fused
// MLP, and residu[i] += ((w0 s0[i] + w1 s1[i]) + ...) in expert order. parties: u64[experts] device
// addresses of the experts' level-0 parts; luts: the layer's u32[3][4][4096]. No host sync: the
// selection flows from the router to the expert kernels through device memory.
extern "C" int trc_couche_moe_fusionnee(trc_vue parties, uint32_t experts, trc_vue luts, const trc_dims_expert* dims,
                                        trc_vue routeur, trc_vue routeur_biais, trc_vue x, uint32_t k,
                                        trc_vue residu, trc_vue indices, trc_vue poids, trc_vue controle,
                                        trc_vue travail, uint32_t n_delta, uint32_t n_codes, void* flux) {
    int r = verifier_forme(dims, n_codes);
    if (r != TRC_OK) return r;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0], D = dims->lignes[2];
    TRC_VERIFIER(dims->lignes[1] == R && dims->colonnes[1] == C && dims->colonnes[2] == R,
                 "gate, up et down incompatibles");
    TRC_VERIFIER(D == C, "la sortie des experts (%u) doit avoir la taille de x (%u)", D, C);
    TRC_VERIFIER(experts > 0 && experts <= 256 && k > 0 && k <= 8 && k <= experts, "top-%u sur %u", k, experts);
    TRC_VERIFIER(n_delta > 0 && n_delta <= 65535, "N de DELTA %u", n_delta);
    TRC_VERIFIER(parties.adresse && parties.octets >= 8ull * experts, "table des parties trop courte");
    TRC_VERIFIER(luts.adresse && luts.octets >= uint64_t(trc::LUTS_PAR_COUCHE) * 4, "LUT trop courtes");
    TRC_VERIFIER(routeur.adresse && routeur.octets >= 2ull * experts * C && routeur.adresse % 8 == 0,
                 "routeur bf16 trop court ou non aligne sur 8");
    TRC_VERIFIER(routeur_biais.adresse == 0 || routeur_biais.octets >= 4ull * experts, "biais du routeur trop court");
    TRC_VERIFIER(x.adresse && x.octets >= 4ull * C && x.adresse % 16 == 0, "x trop court ou non aligne");
    TRC_VERIFIER(residu.adresse && residu.octets >= 4ull * D, "residu trop court");
    TRC_VERIFIER(indices.adresse && indices.octets >= 4ull * k && poids.adresse && poids.octets >= 4ull * k,
                 "indices ou poids trop courts");
    TRC_VERIFIER(controle.adresse && controle.octets >= 16, "controle de moins de 16 o");
    const uint64_t besoin = trc_taille_travail_couche_moe(dims, experts, k, n_codes);
    TRC_VERIFIER(travail.adresse && travail.octets >= besoin && travail.adresse % 256 == 0,
                 "travail de %llu o, %llu o demandes (aligne sur 256)", (unsigned long long)travail.octets,
                 (unsigned long long)besoin);
    const uint32_t Rm = D > R ? D : R;
    const uint32_t Cm = C;
    const uint64_t pas = pas_tache(Rm, Cm, n_codes);
    uint64_t p = travail.adresse;
    const uint64_t t_delta = p;                              // 3k jobs
    const uint64_t t_gu = t_delta + 3ull * k * sizeof(Tache);  // 2k jobs
    const uint64_t t_bas = t_gu + 2ull * k * sizeof(Tache);    // k jobs
    p += al(3ull * k * sizeof(Tache)) * 2;
    const uint64_t logits = p;
    p += al(4ull * experts);
    const uint64_t morceaux = p;
    p += 3ull * k * pas;
    const uint64_t gu = p;
    p += al(4ull * 2 * k * R);
    const uint64_t act = p;
    p += al(4ull * k * R);
    const uint64_t sorties = p;

    const hipStream_t f = flux_de(flux);
    auto ctl = reinterpret_cast<uint32_t*>(controle.adresse);
    const uint32_t* l = reinterpret_cast<const uint32_t*>(luts.adresse);
    TRC_LANCER(fusion_routeur, dim3((experts + 31) / 32), dim3(256), f,
               reinterpret_cast<const uint16_t*>(routeur.adresse), reinterpret_cast<const float*>(x.adresse),
               reinterpret_cast<const float*>(routeur_biais.adresse), reinterpret_cast<float*>(logits), experts, C);
    TRC_LANCER(routeur_topk, dim3(1), dim3(64), f, reinterpret_cast<const float*>(logits), experts, k,
               reinterpret_cast<uint32_t*>(indices.adresse), reinterpret_cast<float*>(poids.adresse),
               static_cast<uint32_t*>(nullptr), 0u);
    trc::ParamsTaches pt;
    pt.parties = parties.adresse;
    pt.indices = indices.adresse;
    pt.x = x.adresse;
    pt.act = act;
    pt.ech = morceaux;
    pt.partiels = morceaux + al(uint64_t(Rm) * (Cm / 32));
    pt.delta = t_delta;
    pt.gu = t_gu;
    pt.bas = t_bas;
    pt.k = k;
    pt.E = experts;
    pt.pas = pas;
    for (int j = 0; j < 3; ++j) {
        pt.lignes[j] = dims->lignes[j];
        pt.colonnes[j] = dims->colonnes[j];
        pt.kmax[j] = kmax_pour(dims->colonnes[j], n_codes);
    }
    TRC_LANCER(fusion_taches, dim3(1), dim3(64), f, pt, ctl);
    const Tache* td = reinterpret_cast<const Tache*>(t_delta);
    const uint32_t B = C / 32;
    TRC_LANCER(fusion_echelles, dim3(grille_tuiles(uint64_t(R) * B, n_delta, 4), 3 * k), dim3(128), f, td, l, ctl);
    TRC_LANCER_N("fusion_gemv/gate_up", fusion_gemv, dim3(grille_tuiles(16ull * R * B, n_codes, 8), 2 * k), dim3(256),
                 f, reinterpret_cast<const Tache*>(t_gu), l, ctl);
    TRC_LANCER(fusion_finir, dim3((R + 255) / 256, 2 * k), dim3(256), f, reinterpret_cast<const Tache*>(t_gu),
               reinterpret_cast<float*>(gu), R);
    TRC_LANCER(fusion_swiglu, dim3((R + 255) / 256, k), dim3(256), f, reinterpret_cast<const float*>(gu),
               reinterpret_cast<float*>(act), R, k);
    TRC_LANCER_N("fusion_gemv/down", fusion_gemv, dim3(grille_tuiles(16ull * D * (R / 32), n_codes, 8), k), dim3(256),
                 f, reinterpret_cast<const Tache*>(t_bas), l, ctl);
    TRC_LANCER(fusion_finir, dim3((D + 255) / 256, k), dim3(256), f, reinterpret_cast<const Tache*>(t_bas),
               reinterpret_cast<float*>(sorties), D);
    TRC_LANCER(combiner, dim3((D + 255) / 256), dim3(256), f, reinterpret_cast<float*>(residu.adresse),
               reinterpret_cast<const float*>(sorties), D, reinterpret_cast<const float*>(poids.adresse), k, D);
    return TRC_OK;
}
