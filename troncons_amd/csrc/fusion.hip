// fusion.hip — the fused expert path for gfx950: rANS decoding of the .trc v1.2 streams feeds the
// MXFP4 dequant and the GEMV directly; decoded code bytes live only in registers and are never
// written to device memory. Kernels, chained on one stream:
//
//   fusion_echelles  DELTA tiles -> E8M0 scales of the selected matrices (a small workspace);
//   fusion_gemv      CODES_CTX tiles -> per-(row, tile) partial sums of y = W x, decoded bytes
//                    dequantised and multiplied in registers;
//   fusion_finir     y[r] = fixed-order sum of the row's tile partials + bias;
//   fusion_swiglu    gpt-oss clamped SwiGLU of the gate/up outputs;
//   fusion_routeur / fusion_taches  (MoE layer) router logits, then the job table of the
//                    selected experts, built on the device from the top-k indices.
//
// Mapping: one wavefront = two rANS tiles (lanes 0-31, 32-63), each tile's words staged in an LDS
// ring (anneau.hpp). In a macro-step, lane v of a tile produces the 4 code bytes 4(v%4) ..
// 4(v%4)+3 of block 8m + v/4, i.e. the weights of columns 32b + 4(v%4) + k (low nibbles) and
// 32b + 16 + 4(v%4) + k (high nibbles): two float4 of x. Each lane accumulates its block
// contributions per row; rows are closed by a 32-lane reduction when the tile's first block enters
// a new row (a row has >= 8 blocks, so one macro-step touches at most two rows). Every (row, tile)
// partial is written exactly once and summed in tile order by the finisher: results are
// deterministic, without floating-point atomics.
#include <hip/hip_runtime.h>

#include <cstring>

#include "anneau.hpp"
#include "chrono.hpp"
#include "commun.hpp"
#include "erreurs.hpp"
#include "fusion_corps.hpp"

// Reference-API kernels (noyaux.hip) reused by the MoE layer.
extern "C" __global__ void routeur_topk(const float* logits, uint32_t E, uint32_t k, uint32_t* indices, float* poids,
                                       uint32_t* boite, uint32_t sequence);
extern "C" __global__ void combiner(float* residu, const float* sorties, uint32_t pas, const float* poids, uint32_t n,
                                    uint32_t d);

// The layer's LUTs u32[3][4][4096] (reference format) are shared by all jobs of a launch.
extern "C" __global__ void __launch_bounds__(trc::FILS_ECHELLES_FUSION)
fusion_echelles(trc::Taches taches, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    __shared__ uint2 lut[trc::M];
    __shared__ uint8_t med[8192];
    __shared__ __attribute__((aligned(16))) uint8_t anneaux[(trc::FILS_ECHELLES_FUSION / 32) * trc::OCTETS_ANNEAU];
    const trc::Tache tc = taches[blockIdx.y];
    trc::etendre_luts(luts + (uint64_t(tc.j) * 4u + 0u) * trc::M, lut, trc::M);
    __syncthreads();
    trc::corps_echelles_fusion(tc, lut, med, anneaux, controle);
}

extern "C" __global__ void __launch_bounds__(trc::FILS_GEMV_FUSION)
fusion_gemv(trc::Taches taches, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    __shared__ uint2 lut[3 * trc::M];
    __shared__ __attribute__((aligned(16))) uint8_t anneaux[(trc::FILS_GEMV_FUSION / 32) * trc::OCTETS_ANNEAU];
    const trc::Tache tc = taches[blockIdx.y];
    trc::etendre_luts(luts + (uint64_t(tc.j) * 4u + 1u) * trc::M, lut, 3u * trc::M);
    __syncthreads();
    trc::corps_gemv_fusion(tc, lut, anneaux, controle);
}

// sorties[y * pas + r] = fixed-order sum of the partials of row r + bias[r], for job y.
extern "C" __global__ void __launch_bounds__(256)
fusion_finir(trc::Taches taches, float* __restrict__ sorties, uint32_t pas) {
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
// 2i+1 (up) in table `gu` against x, job i (down) in table `bas` against act + i*R, and the
// DELTA jobs (3 per expert) in `delta`. Workspace pieces are laid out per (i, j).
namespace trc {
struct ParamsTaches {
    uint64_t parties;   // u64[E] part addresses
    uint64_t indices;   // u32[k]
    uint64_t x;         // f32[C]
    uint64_t act;       // f32[k * R]
    uint64_t ech;       // scales: (i*3 + j) * pas
    uint64_t partiels;  // partials: (i*3 + j) * pas
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

using trc::Tache;
using trc::Taches;
using trc::usage;

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

constexpr uint32_t TUILES_ECHELLES = trc::FILS_ECHELLES_FUSION / 32;
constexpr uint32_t TUILES_GEMV = trc::FILS_GEMV_FUSION / 32;

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

Taches par_valeur(const Tache* t, uint32_t n) {
    Taches l;
    l.table = nullptr;
    for (uint32_t i = 0; i < n && i < 3; ++i) l.locales[i] = t[i];
    return l;
}

Taches par_table(uint64_t adresse) {
    Taches l;
    std::memset(&l, 0, sizeof(l));
    l.table = reinterpret_cast<const Tache*>(adresse);
    return l;
}

}  // namespace

extern "C" uint64_t trc_taille_travail_gemv_fusionnee(uint32_t lignes, uint32_t colonnes, uint32_t n_codes) {
    if (colonnes / 32 < 8 || n_codes == 0) return 0;
    return pas_tache(lignes, colonnes, n_codes);
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
    t.ech = travail.adresse;
    t.partiels = t.ech + al(uint64_t(lignes) * (colonnes / 32));
    t.j = j;
    t.kmax = kmax_pour(colonnes, n_codes);
    t.lignes = lignes;
    t.colonnes = colonnes;
    const Taches tv = par_valeur(&t, 1);
    const hipStream_t f = flux_de(flux);
    auto ctl = reinterpret_cast<uint32_t*>(controle.adresse);
    auto l = reinterpret_cast<const uint32_t*>(luts.adresse);
    const uint32_t B = colonnes / 32;
    TRC_LANCER(fusion_echelles, dim3(grille_tuiles(uint64_t(lignes) * B, n_delta, TUILES_ECHELLES), 1),
               dim3(trc::FILS_ECHELLES_FUSION), f, tv, l, ctl);
    TRC_LANCER(fusion_gemv, dim3(grille_tuiles(16ull * lignes * B, n_codes, TUILES_GEMV), 1),
               dim3(trc::FILS_GEMV_FUSION), f, tv, l, ctl);
    TRC_LANCER(fusion_finir, dim3((lignes + 255) / 256, 1), dim3(256), f, tv, reinterpret_cast<float*>(y.adresse), 0u);
    return TRC_OK;
}

extern "C" uint64_t trc_taille_travail_expert_fusionne(const trc_dims_expert* dims, uint32_t n_codes) {
    if (verifier_forme(dims, n_codes) != TRC_OK) return 0;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0];
    const uint32_t Rm = dims->lignes[2] > R ? dims->lignes[2] : R;
    const uint32_t Cm = dims->colonnes[2] > C ? dims->colonnes[2] : C;
    return 3 * pas_tache(Rm, Cm, n_codes) + al(4ull * 2 * R) + al(4ull * R);
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
    const uint64_t base = travail.adresse;
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
    const Taches trois = par_valeur(t, 3), bas = par_valeur(t + 2, 1);
    const hipStream_t f = flux_de(flux);
    const uint32_t* l = reinterpret_cast<const uint32_t*>(luts.adresse);
    auto ctl = reinterpret_cast<uint32_t*>(controle.adresse);
    const uint32_t B = C / 32;
    TRC_LANCER(fusion_echelles, dim3(grille_tuiles(uint64_t(Rm) * (Cm / 32), n_delta, TUILES_ECHELLES), 3),
               dim3(trc::FILS_ECHELLES_FUSION), f, trois, l, ctl);
    TRC_LANCER(fusion_gemv, dim3(grille_tuiles(16ull * R * B, n_codes, TUILES_GEMV), 2), dim3(trc::FILS_GEMV_FUSION), f,
               trois, l, ctl);
    TRC_LANCER(fusion_finir, dim3((R + 255) / 256, 2), dim3(256), f, trois, reinterpret_cast<float*>(gu), R);
    TRC_LANCER(fusion_swiglu, dim3((R + 255) / 256, 1), dim3(256), f, reinterpret_cast<const float*>(gu),
               reinterpret_cast<float*>(act), R, 1u);
    const uint32_t R2 = dims->lignes[2], B2 = dims->colonnes[2] / 32;
    TRC_LANCER(fusion_gemv, dim3(grille_tuiles(16ull * R2 * B2, n_codes, TUILES_GEMV), 1), dim3(trc::FILS_GEMV_FUSION),
               f, bas, l, ctl);
    TRC_LANCER(fusion_finir, dim3((R2 + 255) / 256, 1), dim3(256), f, bas, reinterpret_cast<float*>(sortie.adresse),
               0u);
    return TRC_OK;
}

extern "C" uint64_t trc_taille_travail_couche_moe(const trc_dims_expert* dims, uint32_t experts, uint32_t k,
                                                  uint32_t n_codes) {
    if (verifier_forme(dims, n_codes) != TRC_OK || k == 0 || k > 8 || experts == 0) return 0;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0];
    const uint32_t Rm = dims->lignes[2] > R ? dims->lignes[2] : R;
    const uint32_t Cm = dims->colonnes[2] > C ? dims->colonnes[2] : C;
    return al(6ull * k * sizeof(Tache)) + al(4ull * experts) + 3ull * k * pas_tache(Rm, Cm, n_codes) +
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
    const uint64_t t_delta = p;                                // 3k jobs
    const uint64_t t_gu = t_delta + 3ull * k * sizeof(Tache);  // 2k jobs
    const uint64_t t_bas = t_gu + 2ull * k * sizeof(Tache);    // k jobs
    p += al(6ull * k * sizeof(Tache));
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
    const uint32_t B = C / 32;
    TRC_LANCER(fusion_echelles, dim3(grille_tuiles(uint64_t(R) * B, n_delta, TUILES_ECHELLES), 3 * k),
               dim3(trc::FILS_ECHELLES_FUSION), f, par_table(t_delta), l, ctl);
    TRC_LANCER_N("fusion_gemv/gate_up", fusion_gemv, dim3(grille_tuiles(16ull * R * B, n_codes, TUILES_GEMV), 2 * k),
                 dim3(trc::FILS_GEMV_FUSION), f, par_table(t_gu), l, ctl);
    TRC_LANCER(fusion_finir, dim3((R + 255) / 256, 2 * k), dim3(256), f, par_table(t_gu), reinterpret_cast<float*>(gu),
               R);
    TRC_LANCER(fusion_swiglu, dim3((R + 255) / 256, k), dim3(256), f, reinterpret_cast<const float*>(gu),
               reinterpret_cast<float*>(act), R, k);
    TRC_LANCER_N("fusion_gemv/down", fusion_gemv, dim3(grille_tuiles(16ull * D * (R / 32), n_codes, TUILES_GEMV), k),
                 dim3(trc::FILS_GEMV_FUSION), f, par_table(t_bas), l, ctl);
    TRC_LANCER(fusion_finir, dim3((D + 255) / 256, k), dim3(256), f, par_table(t_bas), reinterpret_cast<float*>(sorties),
               D);
    TRC_LANCER(combiner, dim3((D + 255) / 256), dim3(256), f, reinterpret_cast<float*>(residu.adresse),
               reinterpret_cast<const float*>(sorties), D, reinterpret_cast<const float*>(poids.adresse), k, D);
    return TRC_OK;
}
