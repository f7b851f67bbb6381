// fusion.hip — the fused expert path for gfx950: rANS decoding of the .trc v1.2 streams feeds the
// MXFP4 dequant and the GEMV directly; decoded code bytes live only in registers and are never
// written to device memory. Kernels, chained on one stream:
//
//   fusion_echelles  DELTA tiles -> E8M0 scales of the selected matrices (a small workspace);
//   fusion_gemv      CODES_CTX tiles -> per-(row, tile) partial sums of y = W x, decoded bytes
//                    dequantised and multiplied in registers;
//   fusion_finir     y[r] = fixed-order sum of the row's tile partials + bias;
//   fusion_finir_swiglu    the same for gate and up, then the gpt-oss clamped SwiGLU (one expert);
//   fusion_codes     (N_codes 16, N_delta 1 or 2) the CODES pass decoding each tile's DELTA itself;
//                    fusion_codes_swiglu, its MoE down form, builds its x (the SwiGLU row) itself;
//   fusion_finir_combiner  the same for the k down products, then the weighted combine;
//   fusion_routeur   (MoE layer) router logits; the first pass after it runs the top-k, and every
//                    later kernel derives its jobs on the device from the chosen indices.
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

#include <algorithm>
#include <cstring>
#include <mutex>

#include "anneau.hpp"
#include "chrono.hpp"
#include "codes.hpp"
#include "commun.hpp"
#include "erreurs.hpp"
#include "fusion_corps.hpp"
#include "selection.hpp"
#include "norme.hpp"
#include "passe.hpp"
#include "scratch.hpp"


// The layer's LUTs u32[3][4][4096] (reference format) are shared by all jobs of a launch. A
// block stages the LUT in LDS (all loads of a batch in flight together), reads its job's matrix,
// then the medians. In a MoE layer (TACHES_MOE_DELTA) every block first runs the router's top-k on
// the logits itself (wavefront 0; the result is deterministic, so all blocks agree) and block
// (0, 0) publishes the indices and weights for the later passes: no block waits for another.
extern "C" __global__ void __launch_bounds__(trc::FILS_ECHELLES_FUSION) __attribute__((amdgpu_waves_per_eu(8)))
fusion_echelles(trc::Taches taches, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    using namespace trc;
    __shared__ uint2 lut[M];
    __shared__ __attribute__((aligned(16))) uint8_t med[MED_LDS_MAX];
    __shared__ __attribute__((aligned(16))) uint8_t anneaux[(FILS_ECHELLES_FUSION / 32) * OCTETS_ANNEAU];
    __shared__ uint32_t choisis[TOPK_MAX];
    __shared__ __attribute__((aligned(16))) float lg[EXPERTS_MAX];
    const bool moe = taches.mode == TACHES_MOE_DELTA;
    const bool prefill = taches.mode == TACHES_PREFILL_DELTA;
    if (prefill && reinterpret_cast<const uint32_t*>(taches.moe.compte)[blockIdx.y / 3u] == 0u) return;
    const uint32_t j_bloc = (moe || prefill) ? blockIdx.y % 3u : min(taches[blockIdx.y].j, 2u);
    ChargeLut<LOT_LUT_ECHELLES> charge_lut;
    charge_lut.demarrer(luts + (uint64_t(j_bloc) * 4u + 0u) * M, M / 4u);
    Tache tc;
    if (moe) {
        // the router's top-k, by ranks over the whole block (selection.hpp); only block (0, 0)
        // computes the weights and publishes the selection for the later passes
        const ParamsMoe& pm = taches.moe;
        const float* logits = reinterpret_cast<const float*>(pm.logits);
        for (uint32_t e = threadIdx.x; e < pm.E; e += blockDim.x) lg[e] = logits[e];
        if (threadIdx.x < TOPK_MAX) choisis[threadIdx.x] = 0xFFFFFFFFu;
        __syncthreads();
        choisir_topk(lg, pm.E, pm.k, choisis, blockDim.x);
        __syncthreads();
        if (blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x < 64u) {
            float w[TOPK_MAX];
            poids_topk(lg, choisis, pm.k, w);
            if (threadIdx.x < pm.k) {
                float wr = w[0];
#pragma unroll
                for (uint32_t r = 1; r < TOPK_MAX; ++r) wr = threadIdx.x == r ? w[r] : wr;
                reinterpret_cast<uint32_t*>(pm.indices)[threadIdx.x] = choisis[threadIdx.x];
                reinterpret_cast<float*>(pm.poids)[threadIdx.x] = wr;
            }
        }
        const uint32_t i = blockIdx.y / 3u;
        tc = uniforme(tache_moe_e(pm, i, blockIdx.y - 3u * i, choisis[i]));
    } else if (prefill) {
        const uint32_t e = blockIdx.y / 3u;
        tc = uniforme(tache_moe_e(taches.moe, e, blockIdx.y - 3u * e, e));
    } else {
        tc = uniforme(taches[blockIdx.y]);
    }
    const MatricePartie m = obtenir_matrice(tc);
    if (moe && blockIdx.x == 0 && threadIdx.x == 0)  // the later passes of the layer read this copy
        ecrire_matrice(reinterpret_cast<void*>(taches.moe.resolus + uint64_t(blockIdx.y) * sizeof(MatricePartie)), m);
    const PrepEchelles p = preparer_echelles(tc, m);
    if (!p.bon) {
        if (threadIdx.x == 0 && blockIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    const TeteTuile tete0 = tete_course(p.h);  // in flight with the medians
    if (tc.lignes <= MED_LDS_MAX) copier_vers_lds(p.fm.p, tc.lignes, p.fm.longueur, med);
    charge_lut.poser(luts + (uint64_t(j_bloc) * 4u + 0u) * M, lut, M / 4u);
    __syncthreads();
    if (tc.lignes <= MED_LDS_MAX)  // uniform
        corps_echelles_fusion<true>(tc, p, lut, med, anneaux, controle, tete0);
    else
        corps_echelles_fusion<false>(tc, p, lut, med, anneaux, controle, tete0);
}

namespace trc {

// residu[r] += ((w0 s0[r] + w1 s1[r]) + w2 s2[r]) + ..., s_i the finished rows of job i, each
// product and sum rounded on its own (the reference combiner, passe.cuh:611-622); s_i is summed as
// somme_fin does, with every job's first two partial sums and bias of the row loaded together.
__device__ __forceinline__ void combiner_lignes(const Fin* fins, uint32_t k, const float* __restrict__ poids,
                                                float* __restrict__ residu, uint32_t D, uint32_t r0, uint32_t pas) {
#pragma clang fp contract(off)
    for (uint32_t r = r0; r < D; r += pas) {
        bool ok = true;
        for (uint32_t i = 0; i < k; ++i) ok = ok && fins[i].bon && r < fins[i].lignes;
        if (!ok) continue;
        const float res = residu[r];
        float p0[TOPK_MAX], p1[TOPK_MAX], bi[TOPK_MAX];
#pragma unroll
        for (uint32_t i = 0; i < TOPK_MAX; ++i) {
            p0[i] = p1[i] = bi[i] = 0.0f;
            if (i < k) {
                // kmax >= 2 for a good job: the second slot of a row is always inside its slots
                const float* p = fins[i].partiels + uint64_t(r) * fins[i].kmax;
                p0[i] = p[0];
                p1[i] = p[1];
                bi[i] = fins[i].biais[r];
            }
        }
        float s = 0.0f;
#pragma unroll
        for (uint32_t i = 0; i < TOPK_MAX; ++i) {
            if (i < k) {
                const Fin& f = fins[i];
                const uint32_t n = partiels_en_plus(f, r);
                float si = p0[i];
                if (n >= 1u) si += p1[i];
                for (uint32_t j = 2; j <= n; ++j) si += f.partiels[uint64_t(r) * f.kmax + j];
                si = si + bi[i];
                const float pr = poids[i] * si;
                s = i == 0 ? pr : s + pr;
            }
        }
        residu[r] = res + s;
    }
}

}  // namespace trc

// CODES pass, x in LDS (colonnes <= X_LDS_MAX): one 160 KiB LDS array laid out as LDS_* says.
extern "C" __global__ void __launch_bounds__(trc::FILS_GEMV_MAX)
fusion_gemv(trc::Taches taches, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    using namespace trc;
    __shared__ __attribute__((aligned(16384))) uint8_t lds[LDS_GEMV];
    const Tache tc = uniforme(taches[blockIdx.y]);
    const uint32_t* lut_src = luts + (uint64_t(min(tc.j, 2u)) * 4u + 1u) * M;
    // Every load that does not depend on the part is issued first: the LUT, and x (16-byte loads of
    // a 16-byte aligned vector of colonnes % 32 == 0 floats; at most 4 per thread, blocks have at
    // least 256 threads and x at most X_LDS_MAX columns), then the matrix record.
    ChargeLut<3> charge_lut;
    charge_lut.demarrer(lut_src, 3u * M / 4u);
    const bool x_lds = tc.colonnes <= X_LDS_MAX;
    const uint32_t n16 = x_lds ? tc.colonnes / 4u : 0u;
    u32x4 xv[4];
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const uint32_t k = threadIdx.x + i * blockDim.x;
        if (k < n16) xv[i] = glob<u32x4>(reinterpret_cast<const void*>(tc.x))[k];
    }
    const PrepGemv p = preparer_gemv(tc, obtenir_matrice(tc));
    const bool bon = p.bon && x_lds;
    // the first tile's head, needed right after the barrier
    const TeteTuile tete0 = bon ? premiere_tete(p.h) : TeteTuile{L, 0u, 0u};
    charge_lut.poser(lut_src, reinterpret_cast<uint2*>(lds + LDS_LUT), 3u * M / 4u);
    if (!bon && threadIdx.x == 0 && blockIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
    if (bon) {
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const uint32_t k = threadIdx.x + i * blockDim.x;
            if (k < n16) *reinterpret_cast<u32x4*>(lds + LDS_X + 16u * k) = xv[i];
        }
        if (threadIdx.x < 8u)  // the zero slot (column block 127) that stream padding blocks read
            *reinterpret_cast<u32x4*>(lds + LDS_X + COLONNE_NULLE * 128u + 16u * threadIdx.x) = u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
    if (bon) corps_gemv_rapide(tc, p, lds, controle, tete0);
}

// CODES pass with each tile's DELTA decoded in the kernel (codes.hpp; streams with N_codes = 16 and
// N_delta 1 or 2), x in LDS. MoE gate/up launches with OPT_TOPK run the router's top-k first (every
// block, by ranks over the logits: the reference's order and tie rule, deterministic, so all blocks
// agree; one wavefront publishes indices and weights), take their expert's matrix from the directory
// and publish the selected experts' three records (resolus) for the down pass and the combine.
// Down launches read x from the experts' SwiGLU rows (fusion_finir_swiglu) or, with SW
// (fusion_codes_swiglu), build it themselves in their prologue.
constexpr uint32_t OPT_TOPK = 2u;
// MoE launches: each CODES block copies its share of its matrix's bias to ParamsMoe::biais (rows
// blockIdx.x * n .. of n = ceil(R / gridDim.x)), the down pass's SwiGLU prologue reads the gate and
// up copies and the combine the down ones: their loads then need no record first.
constexpr uint32_t OPT_BIAIS = 4u;

// SW: the MoE down launch (TACHES_MOE_BAS with OPT_BIAIS); GU: the MoE gate/up launch
// (TACHES_MOE_GU with OPT_TOPK | OPT_BIAIS). Both know their jobs' mode and options at compile time,
// so that no read of them precedes the prologue's first loads.
template <uint32_t FILS, bool SW = false, bool GU = false>
__device__ __forceinline__ void codes_bloc(const trc::Taches& taches, const uint32_t* __restrict__ luts,
                                           uint32_t* __restrict__ controle) {
    using namespace trc;
    __shared__ __attribute__((aligned(16384))) uint8_t lds[LDS_GEMV];
    const Grille g{FILS, uniforme32(gridDim.x)};
    const bool topk = GU || (!SW && (taches.options & OPT_TOPK) != 0u);
    const uint32_t j = SW ? 2u : (topk ? (blockIdx.y & 1u) : min(uniforme32(taches[blockIdx.y].j), 2u));
    const uint32_t* lut_src = luts + (uint64_t(j) * 4u + 1u) * M;
    const ParamsMoe& pm = taches.moe;
    // The prologue is a chain of dependent device-memory reads (logits -> top-k -> the expert's
    // record -> its first tiles' heads -> their words). Everything that does not depend on the
    // top-k's outcome is issued first, unconditionally (indices clamped), in the order it is waited
    // for: the logits; the job's DELTA LUT (staged in LDS for the first tiles' DELTA, its lines also
    // brought into the caches for the later tiles' reads); the decode LUTs; x (its address and
    // width do not depend on the expert).
    const gptr<float> lg_src = glob<float>(topk ? reinterpret_cast<const void*>(pm.logits) : reinterpret_cast<const void*>(luts));
    const float lg_v = lg_src[min(threadIdx.x, (topk ? pm.E : 1u) - 1u)];
    constexpr uint32_t LOT_D = (M / 4u + FILS - 1u) / FILS;  // 16-byte groups of the DELTA LUT per thread
    u32x4 lutd_v[LOT_D];
#pragma unroll
    for (uint32_t k = 0; k < LOT_D; ++k)
        lutd_v[k] = glob<u32x4>(luts + uint64_t(j) * 4u * M)[min(k * FILS + threadIdx.x, M / 4u - 1u)];
    // gate/up: the directory's records of matrix j, one 128-byte line each, so that the one the
    // top-k picks is read from the caches
    const uint32_t rep_chaud =
        glob<uint32_t>(topk ? reinterpret_cast<const void*>(pm.repertoire) : reinterpret_cast<const void*>(luts))
            [topk ? 32u * (3u * min(threadIdx.x, pm.E - 1u) + j) : 0u];
    ChargeLutBloc<FILS> charge_lut;
    charge_lut.demarrer(lut_src);
    const Tache tx = topk ? uniforme(tache_moe_e(pm, blockIdx.y >> 1, j, 0u))
                          : (SW ? uniforme(tache_moe(pm, blockIdx.y, 2u)) : uniforme(taches[blockIdx.y]));
    const bool x_lds = tx.colonnes <= X_LDS_MAX && (SW || tx.x != 0);
    const uint32_t n16 = x_lds ? tx.colonnes / 4u : 0u;
    const gptr<u32x4> x_src = glob<u32x4>(x_lds && !SW ? reinterpret_cast<const void*>(tx.x) : reinterpret_cast<const void*>(luts));
    u32x4 xv[4];
    // SW (MoE down job i): x = swiglu_oai(gate row, up row) of expert i, finished from the gate/up
    // partial sums as fusion_finir_swiglu does (somme_fin, same order, same bits). Rows r = thread +
    // q FILS, q < SW_Q: the partial sums (two per row and matrix: a row spans at most two of the
    // 128-block tiles) are loaded here with the LUTs, the biases once the gate and up records are
    // read, and the SwiGLU is computed while the first tiles' read-ahead is in flight.
    constexpr uint32_t SW_Q = (X_LDS_MAX + FILS - 1u) / FILS;
    const uint32_t i_sw = blockIdx.y;
    const Tache tg = tache_moe(pm, i_sw, 0u), tu = tache_moe(pm, i_sw, 1u);
    const uint32_t R_sw = tx.colonnes;  // gate/up rows = down columns
    u32x2 pg[SW ? SW_Q : 1], pu[SW ? SW_Q : 1];
    float bg[SW ? SW_Q : 1], bu[SW ? SW_Q : 1];
    const bool copies = SW || GU || (taches.options & OPT_BIAIS) != 0u;
    const uint32_t Rm_moe = max(pm.lignes[0], pm.lignes[2]);
    if (SW) {
        // the biases come from the gate/up pass's copies (SW launches carry OPT_BIAIS), loaded here
        // with the partial sums
        const gptr<float> cg = glob<float>(copies ? reinterpret_cast<const void*>(pm.biais + 4ull * (i_sw * 3u) * Rm_moe)
                                                  : reinterpret_cast<const void*>(luts));
        const gptr<float> cu = glob<float>(copies ? reinterpret_cast<const void*>(pm.biais + 4ull * (i_sw * 3u + 1u) * Rm_moe)
                                                  : reinterpret_cast<const void*>(luts));
#pragma unroll
        for (uint32_t q = 0; q < SW_Q; ++q) {
            const uint32_t r = min(threadIdx.x + q * FILS, R_sw - 1u);
            pg[q] = *glob<u32x2>(reinterpret_cast<const void*>(tg.partiels + 8ull * r));
            pu[q] = *glob<u32x2>(reinterpret_cast<const void*>(tu.partiels + 8ull * r));
            bg[q] = cg[copies ? r : 0u];
            bu[q] = cu[copies ? r : 0u];
        }
    } else {
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) xv[i] = x_src[min(threadIdx.x + i * FILS, n16 > 0u ? n16 - 1u : 0u)];
    }
    Tache tc;
    uint32_t e_choisi = 0xFFFFFFFFu;  // topk: the block's chosen expert
    if (topk) {
        // the top-k in the entry area (free until the tiles start)
        // every thread stores its logit (threads past E a copy of logit E - 1, never read): a store
        // under a condition would let the compiler move the logits' load down to it, behind the LUT
        // loads, whose completion the top-k would then wait for
        static_assert(4u * FILS + 4u * TOPK_MAX <= 32u * ENT_PAR_TUILE * 4u, "logits and choices in the entry area");
        float* lg = reinterpret_cast<float*>(lds + LDS_ENT);
        uint32_t* choisis = reinterpret_cast<uint32_t*>(lds + LDS_ENT + 4u * FILS);
        lg[threadIdx.x] = lg_v;
        if (threadIdx.x < TOPK_MAX) choisis[threadIdx.x] = 0xFFFFFFFFu;
        barriere_lds();
        choisir_topk(lg, pm.E, pm.k, choisis, FILS);
        barriere_lds();
        // indices and weights: one wavefront, the last of the first matrix's last block (the tile
        // schedule leaves it without a tile pair when the matrix has fewer pairs than wavefronts),
        // reads the chosen experts and their logits before the barrier and computes the f64 softmax
        // after it, so that no other wavefront waits for it
        const bool poids_ici = blockIdx.y == 0 && blockIdx.x == g.blocs_x - 1u && (threadIdx.x >> 6) == FILS / 64u - 1u;
        uint32_t ch = 0xFFFFFFFFu, ch3 = 0xFFFFFFFFu;
        float choisi[TOPK_MAX];
        if (poids_ici) {  // wave-uniform
            ch = choisis[min(__lane_id(), TOPK_MAX - 1u)];
            ch3 = choisis[min(__lane_id() / 3u, TOPK_MAX - 1u)];
            logits_choisis(lg, choisis, pm.k, choisi);
        }
        const uint32_t i = blockIdx.y >> 1;
        const uint32_t e = uniforme32(choisis[i]);
        // every wave has read the top-k from the entry area before any overwrites it
        barriere_lds();
        if (poids_ici) {
            // the selected experts' records for the later passes: lane l < 3k copies the directory's
            // record (expert l / 3, matrix l % 3) to resolus (the directory is not written during
            // the step; an index past the experts gets a zero record, bon = 0)
            const uint32_t v = __lane_id(), ir = v / 3u, jr = v - 3u * ir;
            if (v < 3u * pm.k) {
                const gptr<u32x4> src = glob<u32x4>(reinterpret_cast<const void*>(
                    pm.repertoire + uint64_t(min(ch3, pm.E - 1u) * 3u + jr) * sizeof(MatricePartie)));
                u32x4 q[sizeof(MatricePartie) / 16u];
#pragma unroll
                for (uint32_t k = 0; k < sizeof(MatricePartie) / 16u; ++k)
                    q[k] = ch3 < pm.E ? src[k] : u32x4{0u, 0u, 0u, 0u};
                typedef __attribute__((address_space(1))) u32x4* GU32X4;
                GU32X4 dst = (GU32X4)(pm.resolus + uint64_t(ir * 3u + jr) * sizeof(MatricePartie));
#pragma unroll
                for (uint32_t k = 0; k < sizeof(MatricePartie) / 16u; ++k) dst[k] = q[k];
            }
            float w[TOPK_MAX];
            poids_de_logits(choisi, pm.k, w);
            if (v < pm.k) {
                float wr = w[0];
#pragma unroll
                for (uint32_t r = 1; r < TOPK_MAX; ++r) wr = v == r ? w[r] : wr;
                typedef __attribute__((address_space(1))) uint32_t* GU32;
                typedef __attribute__((address_space(1))) float* GF32;
                ((GU32)(pm.indices))[v] = ch;
                ((GF32)(pm.poids))[v] = wr;
            }
        }
        tc = uniforme(tache_moe_e(pm, i, j, e));
        e_choisi = e;
    } else {
        tc = tx;
    }
    // SW: the gate and up records' N_codes and check flags, requested with the job's record and
    // checked before the job's (a check after the branch below would let the compiler move their
    // loads down to it, a round trip of their own)
    bool sw_bon = false;
    uint32_t sw_lg = 7u;  // log2 of the gate/up tiles' block count (8 N_codes: 128 or 256)
    MatricePartie mrec;
    if (SW) {
        // the down job's record is a resolved one (never absent), read with the gate and up
        // records' fields in one batch; the checks in bitwise form, so that no branch splits them
        u32x4 gu{lire_u32_constante(tg.matrice + offsetof(MatricePartie, cN)),
                 lire_u32_constante(tg.matrice + offsetof(MatricePartie, bon)),
                 lire_u32_constante(tu.matrice + offsetof(MatricePartie, cN)),
                 lire_u32_constante(tu.matrice + offsetof(MatricePartie, bon))};
        mrec = lire_matrice_groupee(tc.matrice, gu);
        const uint32_t g_cN = gu[0], g_bon = gu[1], u_cN = gu[2], u_bon = gu[3];
        const uint32_t Bg = tg.colonnes / 32u;
        const uint32_t lg = g_cN == 32u ? 8u : 7u;
        sw_bon = (g_bon != 0) & (u_bon != 0) & ((g_cN == 16u) | (g_cN == 32u)) & (u_cN == g_cN) & (Bg >= 8u) &
                 (((Bg - 1u) >> lg) + 2u <= tg.kmax) & (tg.lignes >= R_sw) & (tu.lignes >= R_sw);
        sw_lg = lg;
    } else if (GU) {
        // the chosen expert's record from the directory (an index past the experts, a slot the
        // top-k left empty, reads the last expert's record and fails its checks), in one batch
        u32x4 rien{0u, 0u, 0u, 0u};
        const uint32_t e_mat = uniforme32(min(e_choisi, pm.E - 1u));
        mrec = lire_matrice_groupee(pm.repertoire + uint64_t(e_mat * 3u + j) * sizeof(MatricePartie), rien);
        mrec.bon = e_choisi < pm.E ? mrec.bon : 0u;
    } else {
        mrec = obtenir_matrice_scalaire(tc);
    }
    const PrepCodes p = preparer_codes(tc, mrec);
    const bool bon = p.bon && x_lds && (!SW || (tg.kmax == 2u && copies));  // uniform over the block
    if (!bon) {
        if (threadIdx.x == 0 && blockIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    // the first tile pair's streams (one branch-free batch of loads, left in flight), then x and
    // the decode LUTs into LDS: their loads were issued before, so no wait here drains the
    // read-ahead
    // OPT_BIAIS: this block's share of its matrix's bias, copied after its tiles
    const uint32_t i_moe = topk ? (blockIdx.y >> 1) : blockIdx.y, j_moe = topk ? j : 2u;
    const uint32_t n_copie = (tc.lignes + g.blocs_x - 1u) / g.blocs_x, r_copie = blockIdx.x * n_copie + threadIdx.x;
    const float b_copie = glob<float>(copies ? reinterpret_cast<const void*>(mrec.biais.p) : reinterpret_cast<const void*>(luts))
        [copies ? min(r_copie, tc.lignes - 1u) : 0u];
    // SW: the gate and up records (scalar loads from the resolved records), for their checks
    const Avance avance0 = premiere_avance<true>(p, tc.lignes, g);
    // issued here, ahead of the LDS staging below (which waits on the earlier loads only)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    if (topk) asm volatile("" ::"v"(rep_chaud));  // complete before the decode LUTs, issued after it
    if (SW) {
        const uint32_t Bg = tg.colonnes / 32u;
#pragma unroll
        for (uint32_t q = 0; q < SW_Q; ++q) {
            const uint32_t r = threadIdx.x + q * FILS;
            if (r < R_sw) {
                float v = 0.0f;
                if (sw_bon) {
                    // somme_fin: p[0], + p[1] when the row reaches a second tile, then + bias
                    const bool deux = (r * Bg + Bg - 1u) >> sw_lg != (r * Bg) >> sw_lg;
                    float sg = __uint_as_float(pg[q].x), su = __uint_as_float(pu[q].x);
                    if (deux) {
                        sg += __uint_as_float(pg[q].y);
                        su += __uint_as_float(pu[q].y);
                    }
                    v = swiglu_oai_f(sg + bg[q], su + bu[q]);
                }
                *reinterpret_cast<float*>(lds + LDS_X + 4u * r) = v;
            }
        }
    } else {
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const uint32_t k = threadIdx.x + i * FILS;
            if (k < n16) *reinterpret_cast<u32x4*>(lds + LDS_X + 16u * k) = xv[i];
        }
    }
    if (threadIdx.x < 8u)
        *reinterpret_cast<u32x4*>(lds + LDS_X + COLONNE_NULLE * 128u + 16u * threadIdx.x) = u32x4{0u, 0u, 0u, 0u};
    charge_lut.poser(reinterpret_cast<uint2*>(lds + LDS_LUT));
    // the DELTA LUT copy over the entry area (free since the top-k's last barrier)
#pragma unroll
    for (uint32_t k = 0; k < LOT_D; ++k)
        if (k * FILS + threadIdx.x < M / 4u)
            *reinterpret_cast<u32x4*>(lds + LDS_ENT + 16u * (k * FILS + threadIdx.x)) = lutd_v[k];
    // the block's barriers (LDS only: the read-ahead stays in flight) are passed in corps_codes,
    // around each wavefront's first DELTA decode
    corps_codes(tc, p, lds, luts + uint64_t(j) * 4u * M, controle, avance0, g);
    if (copies && threadIdx.x < n_copie && r_copie < tc.lignes)
        ecrire_global<float>(reinterpret_cast<float*>(pm.biais) + uint64_t(i_moe * 3u + j_moe) * Rm_moe + r_copie, b_copie);
}

extern "C" __global__ void __launch_bounds__(1024)
fusion_codes(trc::Taches taches, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    codes_bloc<1024>(taches, luts, controle);
}
// The MoE gate/up launch with bias copies (TACHES_MOE_GU, OPT_TOPK | OPT_BIAIS), 1024-thread blocks.
extern "C" __global__ void __launch_bounds__(1024)
fusion_codes_gu(trc::Taches taches, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    codes_bloc<1024, false, true>(taches, luts, controle);
}
extern "C" __global__ void __launch_bounds__(512)
fusion_codes_512(trc::Taches taches, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    codes_bloc<512>(taches, luts, controle);
}
extern "C" __global__ void __launch_bounds__(256)
fusion_codes_256(trc::Taches taches, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    codes_bloc<256>(taches, luts, controle);
}
// MoE down pass that builds its x (the SwiGLU of expert blockIdx.y's gate and up rows) itself.
extern "C" __global__ void __launch_bounds__(1024)
fusion_codes_swiglu(trc::Taches taches, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    codes_bloc<1024, true>(taches, luts, controle);
}

// The CODES kernel compiled for the launch's block size (1024, 512 or 256 threads).
#define TRC_LANCER_CODES(nom, forme, f, ...)                                                     \
    do {                                                                                         \
        if ((forme).bloc.x == 1024)                                                              \
            TRC_LANCER_N(nom, fusion_codes, (forme).grille, (forme).bloc, f, __VA_ARGS__);       \
        else if ((forme).bloc.x == 512)                                                          \
            TRC_LANCER_N(nom, fusion_codes_512, (forme).grille, (forme).bloc, f, __VA_ARGS__);   \
        else                                                                                     \
            TRC_LANCER_N(nom, fusion_codes_256, (forme).grille, (forme).bloc, f, __VA_ARGS__);   \
    } while (0)

// CODES pass, x read from device memory (rows of any width).
extern "C" __global__ void __launch_bounds__(trc::FILS_GEMV_MAX)
fusion_gemv_xg(trc::Taches taches, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    using namespace trc;
    __shared__ uint2 lut[3 * M];
    __shared__ __attribute__((aligned(16))) uint8_t anneaux[(FILS_GEMV_MAX / 32) * OCTETS_ANNEAU];
    __shared__ __attribute__((aligned(16))) uint32_t ent[(FILS_GEMV_MAX / 32) * ENT_PAR_TUILE];
    const Tache tc = uniforme(taches[blockIdx.y]);
    etendre_luts<3>(luts + (uint64_t(min(tc.j, 2u)) * 4u + 1u) * M, lut, 3u * M / 4u);
    const PrepGemv p = preparer_gemv(tc, obtenir_matrice(tc));
    if (!p.bon) {
        if (threadIdx.x == 0 && blockIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    __syncthreads();
    corps_gemv_xg(tc, p, lut, anneaux, ent, controle);
}

// ---------------------------------------------------------------------------------- finishers

// sorties[y * pas + r] = fixed-order sum of the partials of row r + bias[r], for job y.
extern "C" __global__ void __launch_bounds__(256)
fusion_finir(trc::Taches taches, float* __restrict__ sorties, uint32_t pas) {
    using namespace trc;
    __shared__ Fin fins[1];
    preparer_fins(taches, blockIdx.y, 1, fins);
    const Fin f = fins[0];
    const uint32_t r = blockIdx.x * 256u + threadIdx.x;
    if (!f.bon || r >= f.lignes) return;  // format errors are counted by fusion_gemv
    sorties[uint64_t(blockIdx.y) * pas + r] = somme_fin(f, r);
}

// act[i*R + r] = swiglu_oai(gate_i[r], up_i[r]) with gate_i, up_i the finished rows of jobs 2i and
// 2i+1 (gpt-oss clamped SwiGLU in f64, one rounding: the reference swiglu_oai, passe.cuh:598-605).
extern "C" __global__ void __launch_bounds__(256)
fusion_finir_swiglu(trc::Taches taches, float* __restrict__ act, uint32_t R) {
    using namespace trc;
    __shared__ Fin fins[2];
    const uint32_t i = blockIdx.y;
    preparer_fins(taches, 2u * i, 2, fins);
    const uint32_t r = blockIdx.x * 256u + threadIdx.x;
    if (!fins[0].bon || !fins[1].bon || r >= R || r >= fins[0].lignes || r >= fins[1].lignes) return;
    act[uint64_t(i) * R + r] = swiglu_oai_f(somme_fin(fins[0], r), somme_fin(fins[1], r));
}

// residu[r] += ((w0 s0[r] + w1 s1[r]) + w2 s2[r]) + ... over the k down jobs (MoE layer).
// OPT_BIAIS (one row per thread, 2 partial-sum slots per row): the row's residual, partial sums and
// bias copies are loaded before the records' fields are read (scalar loads), so that both take one
// round trip.
extern "C" __global__ void __launch_bounds__(256)
fusion_finir_combiner(trc::Taches taches) {
    using namespace trc;
    __shared__ Fin fins[TOPK_MAX];
    const ParamsMoe& moe = taches.moe;
    if ((taches.options & OPT_BIAIS) != 0u) {
        // KM: the jobs loaded per row, 4 for a top-4 (or less) layer, else TOPK_MAX
        auto combiner = [&](auto km) {
#pragma clang fp contract(off)
            constexpr uint32_t KM = decltype(km)::value;
            const uint32_t D = moe.lignes[2], Rm = max(moe.lignes[0], moe.lignes[2]);
            const uint32_t r = blockIdx.x * 256u + threadIdx.x, rr = min(r, D - 1u);
            const float res = glob<float>(reinterpret_cast<const void*>(moe.residu))[rr];
            u32x2 p[KM];
            float bi[KM], w[KM];
#pragma unroll
            for (uint32_t i = 0; i < KM; ++i) {
                const uint32_t ii = min(i, moe.k - 1u);
                p[i] = *glob<u32x2>(reinterpret_cast<const void*>(tache_moe(moe, ii, 2u).partiels + 8ull * rr));
                bi[i] = glob<float>(reinterpret_cast<const void*>(moe.biais))[uint64_t(ii * 3u + 2u) * Rm + rr];
                w[i] = glob<float>(reinterpret_cast<const void*>(moe.poids))[ii];
            }
            // the selected down records' N_codes and check flag (written by the gate/up launch), read
            // with scalar loads into registers, all issued before any is used (the empty asm takes
            // them all, so one wait covers them); the checks in bitwise form, one return: no LDS copy
            // of the records, no barrier, no round trip per job
            uint32_t cn[KM], bn[KM];
#pragma unroll
            for (uint32_t i = 0; i < KM; ++i) {
                const uint64_t rec = tache_moe(moe, min(i, moe.k - 1u), 2u).matrice;
                cn[i] = lire_u32_constante(rec + offsetof(MatricePartie, cN));
                bn[i] = lire_u32_constante(rec + offsetof(MatricePartie, bon));
            }
#pragma unroll
            for (uint32_t i = 0; i < KM; ++i) asm volatile("" : "+s"(cn[i]), "+s"(bn[i]));
            Fin f[KM];
            bool ok = r < D;
#pragma unroll
            for (uint32_t i = 0; i < KM; ++i) {
                const Tache t = tache_moe(moe, min(i, moe.k - 1u), 2u);
                f[i].B = t.colonnes / 32u;
                f[i].bpt = 8u * max(cn[i], 1u);
                f[i].kmax = t.kmax;
                f[i].lignes = t.lignes;
                // (B - 1) / bpt + 2 <= kmax, without the division
                f[i].bon = (bn[i] != 0u) & (f[i].B >= 8u) & (t.kmax >= 2u) & (f[i].B - 1u < (t.kmax - 1u) * f[i].bpt);
                ok &= (i >= moe.k) | (f[i].bon & (r < f[i].lignes) & (f[i].kmax == 2u));
            }
            if (!ok) return;
            float s = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < KM; ++i) {
                if (i < moe.k) {
                    float si = __uint_as_float(p[i].x);
                    if (partiels_en_plus(f[i], r) >= 1u) si += __uint_as_float(p[i].y);
                    si = si + bi[i];
                    const float pr = w[i] * si;
                    s = i == 0 ? pr : s + pr;
                }
            }
            ecrire_global<float>(reinterpret_cast<float*>(moe.residu) + r, res + s);
        };
        if (moe.k <= 4u)  // uniform
            combiner(std::integral_constant<uint32_t, 4>{});
        else
            combiner(std::integral_constant<uint32_t, TOPK_MAX>{});
        return;
    }
    preparer_fins(taches, 0, moe.k, fins);
    combiner_lignes(fins, moe.k, reinterpret_cast<const float*>(moe.poids), reinterpret_cast<float*>(moe.residu),
                    moe.lignes[2], blockIdx.x * 256u + threadIdx.x, gridDim.x * 256u);
}

// ---------------------------------------------------------------------------- router + top-k
// Router logits y = W x (+ b), W bf16 row-major (E x C), in the reference gemv_f32 order (bf16 ->
// f32 is exact, so the bits equal gemv_f32 on the widened matrix, passe.cuh:104-130): one row per
// half-wavefront, lane v taking float4 groups v, v+32, ...; a row's loads are all in flight while
// the block stages x in LDS. The top-k runs at the start of the DELTA pass.
// With NORME (x then the raw residual), the block stages RMSNorm(x) with `norme` (norme_ligne: the
// rmsnorm kernel's bits) instead of x, and block 0 writes it to h2 for the later passes.
template <bool X_LDS, bool NORME = false>
__device__ __forceinline__ void routeur_lignes(const uint16_t* __restrict__ W, const float* __restrict__ x,
                                               const float* __restrict__ biais, float* __restrict__ y, uint32_t R,
                                               uint32_t C, trc::f32x4* xs, const float* __restrict__ norme = nullptr,
                                               float eps = 0.0f, float* __restrict__ h2 = nullptr) {
    using namespace trc;
    constexpr uint32_t LOT = 24;
    const uint32_t voie = threadIdx.x & 31u;
    const uint32_t r = blockIdx.x * (blockDim.x >> 5) + (threadIdx.x >> 5);
    const uint32_t C4 = C / 4u;
    const gptr<u32x2> W4 = glob<u32x2>(W + uint64_t(min(r, R - 1u)) * C);
    const gptr<f32x4> xg = glob<f32x4>(x);
    u32x2 w[LOT];
#pragma unroll
    for (uint32_t i = 0; i < LOT; ++i)
        if (32u * i + voie < C4) w[i] = W4[32u * i + voie];
    if (NORME) {
        __shared__ double part[FILS_NORME];
        __shared__ double total;
        norme_ligne(x, norme, reinterpret_cast<float*>(xs), C, eps, part, &total);
        __syncthreads();
        if (blockIdx.x == 0)
            for (uint32_t i = threadIdx.x; i < C4; i += blockDim.x) reinterpret_cast<f32x4*>(h2)[i] = xs[i];
    } else if (X_LDS) {
        // every load of x first, then the stores: one round trip (C <= X_LDS_MAX, 256 threads)
        constexpr uint32_t NX = (X_LDS_MAX / 4u + 255u) / 256u;
        f32x4 xv[NX];
#pragma unroll
        for (uint32_t k = 0; k < NX; ++k) xv[k] = xg[min(threadIdx.x + 256u * k, C4 - 1u)];
#pragma unroll
        for (uint32_t k = 0; k < NX; ++k)
            if (threadIdx.x + 256u * k < C4) xs[threadIdx.x + 256u * k] = xv[k];
        __syncthreads();
    }
    float acc = 0.0f;
    for (uint32_t c0 = 0; c0 < C4; c0 += 32u * LOT) {
        if (c0 > 0) {
#pragma unroll
            for (uint32_t i = 0; i < LOT; ++i)
                if (c0 + 32u * i + voie < C4) w[i] = W4[c0 + 32u * i + voie];
        }
#pragma unroll
        for (uint32_t i = 0; i < LOT; ++i) {
            const uint32_t c = c0 + 32u * i + voie;
            if (c < C4) {
                const f32x4 xv = X_LDS || NORME ? xs[c] : f32x4(xg[c]);
                acc = fmaf(__uint_as_float(w[i].x << 16), xv.x, acc);
                acc = fmaf(__uint_as_float(w[i].x & 0xFFFF0000u), xv.y, acc);
                acc = fmaf(__uint_as_float(w[i].y << 16), xv.z, acc);
                acc = fmaf(__uint_as_float(w[i].y & 0xFFFF0000u), xv.w, acc);
            }
        }
    }
    const float s = somme_demi_f32(acc);
    if (voie == 0 && r < R) y[r] = biais != nullptr ? s + biais[r] : s;
}

extern "C" __global__ void __launch_bounds__(256)
fusion_routeur(const uint16_t* __restrict__ W, const float* __restrict__ x, const float* __restrict__ biais,
               float* __restrict__ logits, uint32_t E, uint32_t C) {
    using namespace trc;
    __shared__ f32x4 xs[X_LDS_MAX / 4];
    if (C <= X_LDS_MAX)
        routeur_lignes<true>(W, x, biais, logits, E, C, xs);
    else
        routeur_lignes<false>(W, x, biais, logits, E, C, xs);
}

// The router over RMSNorm(residual) (C <= X_LDS_MAX): the decode step's post-attention norm folded
// into the router; block 0 leaves the normed row in h2 for the DELTA and GEMV passes.
extern "C" __global__ void __launch_bounds__(256)
fusion_routeur_norme(const uint16_t* __restrict__ W, const float* __restrict__ residu, const float* __restrict__ norme,
                     float eps, float* __restrict__ h2, const float* __restrict__ biais, float* __restrict__ logits,
                     uint32_t E, uint32_t C) {
    using namespace trc;
    static_assert(FILS_NORME == 256, "one router block runs the norm");
    __shared__ f32x4 xs[X_LDS_MAX / 4];
    routeur_lignes<true, true>(W, residu, biais, logits, E, C, xs, norme, eps, h2);
}

// ---------------------------------------------------------------------------------- layer mount
// Directory of a resident layer: for expert e (block x) and matrix j (block y), one wavefront walks
// the part once and writes its MatricePartie to repertoire[e*3 + j]; a part that fails a check gets
// bon = 0 there and one format error in controle (every later use of it counts one more).
extern "C" __global__ void __launch_bounds__(64)
fusion_monter(const uint64_t* __restrict__ parties, trc_dims_expert dims, trc::MatricePartie* __restrict__ repertoire,
              uint32_t* __restrict__ controle) {
    using namespace trc;
    const uint32_t e = blockIdx.x, j = blockIdx.y;
    const uint8_t* partie = reinterpret_cast<const uint8_t*>(uniforme64(parties[e]));
    const MatricePartie m = analyser_matrice(partie, j, choisir(dims.lignes, j), choisir(dims.colonnes, j));
    if (threadIdx.x == 0) {
        ecrire_matrice(repertoire + uint64_t(e) * 3u + j, m);
        if (!m.bon) atomicAdd(&controle[CTL_FORMAT], 1u);
    }
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

// Grid of a DELTA pass over `travaux` matrices of `blocs` blocks: each half-wavefront takes a run of
// whole tiles, so that a block's prologue (LUT, record, medians, top-k) and a ring's opening serve
// several tiles; runs of about 32 macro-steps when the launch has work for more than 8192
// half-wavefronts (a 1024-thread block per CU) at that length, shorter ones down to a single tile
// when it has less, so that a small launch (one token's matrices) keeps its parallelism.
uint32_t grille_echelles(uint64_t blocs, uint32_t n_delta, uint32_t travaux) {
    const uint32_t n = n_delta ? n_delta : 1u;
    const uint64_t par_demi = ((blocs + 127u) / 128u) * travaux / 8192u;  // macro-steps per half at 8192 halves
    const uint64_t tuiles = std::min<uint64_t>(std::max<uint64_t>(par_demi / n, 1u), n < 32u ? 32u / n : 1u);
    return grille_tuiles(blocs, uint32_t(n * tuiles), TUILES_ECHELLES);
}

// Workspace of one matrix job: block entries (u32 per block + staging margin), then partial sums.
uint64_t octets_ech(uint32_t R, uint32_t C) { return al(4ull * (uint64_t(R) * (C / 32) + trc::ECH_MARGE)); }

uint64_t pas_tache(uint32_t R, uint32_t C, uint32_t n_codes) {
    return octets_ech(R, C) + al(4ull * R * kmax_pour(C, n_codes));
}

// The CODES pass decodes each tile's DELTA itself (fusion_codes, codes.hpp) for streams of 16
// macro-steps per CODES tile and 1 or 2 per DELTA tile, or 32 and 2: no DELTA launch, no block
// entries. In that plan each matrix may take either form (the kernels read N from its streams).
// Other tile lengths take the DELTA pass, whose block entries go through the workspace.
bool delta_interne(uint32_t n_delta, uint32_t n_codes) { return trc::delta_dans_codes(n_delta, n_codes); }

// Workspace piece of one matrix job in the internal-DELTA mode: its partial sums only.
uint64_t pas_tache_interne(uint32_t R, uint32_t C) { return al(4ull * R * kmax_pour(C, 16)); }

// Launch shape of a CODES pass over `jobs` matrices of R x C: 1024, 512 or 256 threads (32, 16 or 8
// tiles) per block, the largest that still gives every CU of the chip a block, and at most about one
// block per CU over all jobs (a block's LDS holds the three LUTs, so one fits a CU): wavefronts then
// loop over further tile pairs instead of new blocks paying the LUT staging and the header reads.
constexpr uint32_t CUS = 256;

struct FormeGemv {
    dim3 grille, bloc;
    bool x_lds;
};

FormeGemv forme_gemv(uint32_t R, uint32_t C, uint32_t N, uint32_t jobs) {
    const uint64_t octets = 16ull * R * (C / 32);
    const uint64_t T = ((octets + 127) / 128 + N - 1) / N;
    uint32_t fils = trc::FILS_GEMV_MAX;
    while (fils > 256 && ((T + fils / 32 - 1) / (fils / 32)) * jobs < CUS) fils /= 2;
    uint32_t gx = grille_tuiles(octets, N, fils / 32);
    const uint32_t plafond = (CUS + jobs - 1) / jobs;
    if (gx > plafond) gx = plafond;
    FormeGemv f;
    f.grille = dim3(gx, jobs);
    f.bloc = dim3(fils);
    f.x_lds = C <= trc::X_LDS_MAX;
    return f;
}

#define TRC_LANCER_GEMV(nom, forme, f, ...)                                                         \
    do {                                                                                            \
        if ((forme).x_lds)                                                                          \
            TRC_LANCER_N(nom, fusion_gemv, (forme).grille, (forme).bloc, f, __VA_ARGS__);           \
        else                                                                                        \
            TRC_LANCER_N(nom "/xg", fusion_gemv_xg, (forme).grille, (forme).bloc, f, __VA_ARGS__); \
    } while (0)

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
    std::memset(&l, 0, sizeof(l));
    l.mode = trc::TACHES_LOCALES;
    for (uint32_t i = 0; i < n && i < 3; ++i) l.locales[i] = t[i];
    return l;
}

Taches par_moe(const trc::ParamsMoe& pm, uint32_t mode, uint32_t options) {
    Taches l;
    std::memset(&l, 0, sizeof(l));
    l.moe = pm;
    l.mode = mode;
    l.options = options;
    return l;
}

}  // namespace

namespace trc {
// DELTA pass of a batched prefill (prefill.hip): matrices (e, j) of every expert with compte[e] > 0,
// block entries into workspace piece e*3 + j.
int lancer_echelles_prefill(const ParamsMoe& pm, uint32_t R, uint32_t C, uint32_t n_delta, const uint32_t* luts,
                            uint32_t* ctl, hipStream_t f) {
    const Taches t = par_moe(pm, TACHES_PREFILL_DELTA, 0);
    TRC_LANCER_N("fusion_echelles/prefill", fusion_echelles,
                 dim3(grille_echelles(uint64_t(R) * (C / 32), n_delta, 3 * pm.E), 3 * pm.E),
                 dim3(FILS_ECHELLES_FUSION), f, t, luts, ctl);
    return TRC_OK;
}
uint64_t octets_entrees(uint32_t R, uint32_t C) { return octets_ech(R, C); }
}  // namespace trc

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
    TRC_VERIFIER(partie.adresse && partie.octets >= 64 && partie.adresse % 16 == 0,
                 "partie trop courte ou non alignee sur 16");
    TRC_VERIFIER(luts.adresse && luts.octets >= uint64_t(trc::LUTS_PAR_COUCHE) * 4, "LUT trop courtes");
    TRC_VERIFIER(x.adresse && x.octets >= 4ull * colonnes && x.adresse % 16 == 0, "x trop court ou non aligne");
    TRC_VERIFIER(y.adresse && y.octets >= 4ull * lignes, "y trop court");
    TRC_VERIFIER(controle.adresse && controle.octets >= 16, "controle de moins de 16 o");
    const uint64_t besoin = trc_taille_travail_gemv_fusionnee(lignes, colonnes, n_codes);
    TRC_VERIFIER(travail.adresse && travail.octets >= besoin && travail.adresse % 256 == 0,
                 "travail de %llu o, %llu o demandes (aligne sur 256)", (unsigned long long)travail.octets,
                 (unsigned long long)besoin);
    Tache t{};
    t.partie = partie.adresse;
    t.x = x.adresse;
    t.ech = travail.adresse;
    t.partiels = t.ech + octets_ech(lignes, colonnes);
    t.j = j;
    t.kmax = kmax_pour(colonnes, n_codes);
    t.lignes = lignes;
    t.colonnes = colonnes;
    const hipStream_t f = flux_de(flux);
    auto ctl = reinterpret_cast<uint32_t*>(controle.adresse);
    auto l = reinterpret_cast<const uint32_t*>(luts.adresse);
    const uint32_t B = colonnes / 32;
    if (delta_interne(n_delta, n_codes) && colonnes <= trc::X_LDS_MAX) {
        t.ech = 0;
        t.partiels = travail.adresse;
        const Taches tv = par_valeur(&t, 1);
        const FormeGemv fo = forme_gemv(lignes, colonnes, n_codes, 1);
        TRC_LANCER_CODES("fusion_codes", fo, f, tv, l, ctl);
        TRC_LANCER(fusion_finir, dim3((lignes + 255) / 256, 1), dim3(256), f, tv, reinterpret_cast<float*>(y.adresse), 0u);
        return TRC_OK;
    }
    const Taches tv = par_valeur(&t, 1);
    TRC_LANCER(fusion_echelles, dim3(grille_echelles(uint64_t(lignes) * B, n_delta, 1), 1),
               dim3(trc::FILS_ECHELLES_FUSION), f, tv, l, ctl);
    TRC_LANCER_GEMV("fusion_gemv", forme_gemv(lignes, colonnes, n_codes, 1), f, tv, l, ctl);
    TRC_LANCER(fusion_finir, dim3((lignes + 255) / 256, 1), dim3(256), f, tv, reinterpret_cast<float*>(y.adresse), 0u);
    return TRC_OK;
}

extern "C" uint64_t trc_taille_travail_expert_fusionne(const trc_dims_expert* dims, uint32_t n_codes) {
    if (verifier_forme(dims, n_codes) != TRC_OK) return 0;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0];
    const uint32_t Rm = dims->lignes[2] > R ? dims->lignes[2] : R;
    const uint32_t Cm = dims->colonnes[2] > C ? dims->colonnes[2] : C;
    return 3 * pas_tache(Rm, Cm, n_codes) + al(4ull * R);
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
    TRC_VERIFIER(partie.adresse && partie.octets >= 64 && partie.adresse % 16 == 0,
                 "partie trop courte ou non alignee sur 16");
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
    const uint64_t act = base + 3 * pas;
    Tache t[3] = {};
    for (uint32_t j = 0; j < 3; ++j) {
        t[j].partie = partie.adresse;
        t[j].j = j;
        t[j].lignes = dims->lignes[j];
        t[j].colonnes = dims->colonnes[j];
        t[j].kmax = kmax_pour(dims->colonnes[j], n_codes);
        t[j].ech = base + j * pas;
        t[j].partiels = t[j].ech + octets_ech(Rm, Cm);
        t[j].x = j < 2 ? x.adresse : act;
    }
    const hipStream_t f = flux_de(flux);
    const uint32_t* l = reinterpret_cast<const uint32_t*>(luts.adresse);
    auto ctl = reinterpret_cast<uint32_t*>(controle.adresse);
    if (delta_interne(n_delta, n_codes) && Cm <= trc::X_LDS_MAX) {
        const uint64_t pi = pas_tache_interne(Rm, Cm);
        for (uint32_t j = 0; j < 3; ++j) {
            t[j].ech = 0;
            t[j].partiels = base + j * pi;
        }
        const Taches deux = par_valeur(t, 2), bas = par_valeur(t + 2, 1);
        const FormeGemv fgu = forme_gemv(R, C, n_codes, 2);
        TRC_LANCER_CODES("fusion_codes", fgu, f, deux, l, ctl);
        TRC_LANCER(fusion_finir_swiglu, dim3((R + 255) / 256, 1), dim3(256), f, deux, reinterpret_cast<float*>(act), R);
        const uint32_t R2 = dims->lignes[2];
        const FormeGemv fb = forme_gemv(R2, dims->colonnes[2], n_codes, 1);
        TRC_LANCER_CODES("fusion_codes", fb, f, bas, l, ctl);
        TRC_LANCER(fusion_finir, dim3((R2 + 255) / 256, 1), dim3(256), f, bas,
                   reinterpret_cast<float*>(sortie.adresse), 0u);
        return TRC_OK;
    }
    const Taches trois = par_valeur(t, 3), bas = par_valeur(t + 2, 1);
    TRC_LANCER(fusion_echelles, dim3(grille_echelles(uint64_t(Rm) * (Cm / 32), n_delta, 3), 3),
               dim3(trc::FILS_ECHELLES_FUSION), f, trois, l, ctl);
    TRC_LANCER_GEMV("fusion_gemv", forme_gemv(R, C, n_codes, 2), f, trois, l, ctl);
    TRC_LANCER(fusion_finir_swiglu, dim3((R + 255) / 256, 1), dim3(256), f, trois, reinterpret_cast<float*>(act), R);
    const uint32_t R2 = dims->lignes[2];
    TRC_LANCER_GEMV("fusion_gemv", forme_gemv(R2, dims->colonnes[2], n_codes, 1), f, bas, l, ctl);
    TRC_LANCER(fusion_finir, dim3((R2 + 255) / 256, 1), dim3(256), f, bas, reinterpret_cast<float*>(sortie.adresse),
               0u);
    return TRC_OK;
}

extern "C" uint64_t trc_taille_repertoire(uint32_t experts) {
    return uint64_t(experts) * 3u * sizeof(trc::MatricePartie);
}

// Mounts a resident layer: parses the level-0 part of each of `experts` experts (u64[experts]
// device addresses, 16-byte aligned) once into the directory that trc_couche_moe_fusionnee reads.
extern "C" int trc_monter_couche(trc_vue parties, uint32_t experts, const trc_dims_expert* dims, trc_vue repertoire,
                                 trc_vue controle, void* flux) {
    if (dims == nullptr) return usage("dims absent");
    int r = trc_dims_verifier(dims);
    if (r != TRC_OK) return r;
    TRC_VERIFIER(experts > 0 && experts <= trc::EXPERTS_MAX, "%u experts", experts);
    TRC_VERIFIER(parties.adresse && parties.octets >= 8ull * experts && parties.adresse % 8 == 0,
                 "table des parties trop courte");
    TRC_VERIFIER(repertoire.adresse && repertoire.octets >= trc_taille_repertoire(experts) &&
                     repertoire.adresse % 16 == 0,
                 "repertoire trop court ou non aligne sur 16");
    TRC_VERIFIER(controle.adresse && controle.octets >= 16, "controle de moins de 16 o");
    TRC_LANCER(fusion_monter, dim3(experts, 3), dim3(64), flux_de(flux),
               reinterpret_cast<const uint64_t*>(parties.adresse), *dims,
               reinterpret_cast<trc::MatricePartie*>(repertoire.adresse), reinterpret_cast<uint32_t*>(controle.adresse));
    return TRC_OK;
}

extern "C" uint64_t trc_taille_travail_couche_moe(const trc_dims_expert* dims, uint32_t experts, uint32_t k,
                                                  uint32_t n_codes) {
    if (verifier_forme(dims, n_codes) != TRC_OK || k == 0 || k > trc::TOPK_MAX || experts == 0) return 0;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0];
    const uint32_t Rm = dims->lignes[2] > R ? dims->lignes[2] : R;
    const uint32_t Cm = dims->colonnes[2] > C ? dims->colonnes[2] : C;
    return al(4ull * experts) + al(3ull * k * sizeof(trc::MatricePartie)) + al(4ull * k * R) + al(12ull * k * Rm) +
           3ull * k * pas_tache(Rm, Cm, n_codes);
}

// Config 3: one MoE layer decode step at batch 1. logits = W_r x (+ b_r) (W_r bf16, experts x C),
// top-k with softmax weights (indices/poids written out), then for the k selected experts the fused
// MLP, and residu[i] += ((w0 s0[i] + w1 s1[i]) + ...) in expert order. repertoire: the layer's
// directory (trc_monter_couche; the parts it points into stay resident); luts: the layer's
// u32[3][4][4096]. No host sync: the selection flows from the router to the expert kernels through
// device memory, and every kernel derives its jobs from the top-k indices (checked against
// `experts` before the directory is read). Streams of 16 macro-steps per CODES tile and 1 or 2 per
// DELTA tile take four launches: router logits; gate/up CODES pass (2k jobs, each block running the
// top-k first, each tile's DELTA decoded in the kernel); down CODES pass (k, each block building its
// x, the expert's SwiGLU row, from the gate/up partial sums in its prologue); finish + combine.
// With down blocks under 1024 threads (or a block's share of bias rows past its threads) the k SwiGLU
// rows take a launch of their own before down.
// Other tile lengths add a DELTA pass (3k matrices, with the top-k) before the gate/up pass. No
// cross-block synchronisation inside a launch. Rows are limited to X_LDS_MAX columns (x in LDS).
namespace {
// The fused MoE layer; with `norme`, the router takes RMSNorm(residu) with `norme` into x first
// (x is then written, not read, by the router).
int couche_moe(trc_vue repertoire, uint32_t experts, trc_vue luts, const trc_dims_expert* dims, trc_vue routeur,
               trc_vue routeur_biais, trc_vue x, uint32_t k, trc_vue residu, trc_vue indices, trc_vue poids,
               trc_vue controle, trc_vue travail, uint32_t n_delta, uint32_t n_codes, trc_vue norme, float eps,
               void* flux) {
    int r = verifier_forme(dims, n_codes);
    if (r != TRC_OK) return r;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0], D = dims->lignes[2];
    TRC_VERIFIER(dims->lignes[1] == R && dims->colonnes[1] == C && dims->colonnes[2] == R,
                 "gate, up et down incompatibles");
    TRC_VERIFIER(D == C, "la sortie des experts (%u) doit avoir la taille de x (%u)", D, C);
    TRC_VERIFIER(experts > 0 && experts <= trc::EXPERTS_MAX && k > 0 && k <= trc::TOPK_MAX && k <= experts,
                 "top-%u sur %u", k, experts);
    TRC_VERIFIER(n_delta > 0 && n_delta <= 65535, "N de DELTA %u", n_delta);
    TRC_VERIFIER(repertoire.adresse && repertoire.octets >= trc_taille_repertoire(experts) &&
                     repertoire.adresse % 16 == 0,
                 "repertoire trop court ou non aligne sur 16");
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
    TRC_VERIFIER(C <= trc::X_LDS_MAX && R <= trc::X_LDS_MAX, "couche de %u x %u : au plus %u colonnes", R, C,
                 trc::X_LDS_MAX);
    const uint32_t Rm = D > R ? D : R;
    const uint32_t Cm = C;
    const uint64_t pas = pas_tache(Rm, Cm, n_codes);
    uint64_t p = travail.adresse;
    const uint64_t logits = p;
    p += al(4ull * experts);
    const uint64_t resolus = p;
    p += al(3ull * k * sizeof(trc::MatricePartie));
    const uint64_t act = p;
    p += al(4ull * k * R);
    const uint64_t biais = p;
    p += al(12ull * k * Rm);
    const uint64_t morceaux = p;

    trc::ParamsMoe pm;
    std::memset(&pm, 0, sizeof(pm));
    pm.repertoire = repertoire.adresse;
    pm.resolus = resolus;
    pm.logits = logits;
    pm.indices = indices.adresse;
    pm.poids = poids.adresse;
    pm.x = x.adresse;
    pm.residu = residu.adresse;
    pm.ech = morceaux;
    pm.partiels = morceaux + octets_ech(Rm, Cm);
    pm.pas = pas;
    pm.k = k;
    pm.E = experts;
    for (int j = 0; j < 3; ++j) {
        pm.lignes[j] = dims->lignes[j];
        pm.colonnes[j] = dims->colonnes[j];
        pm.kmax[j] = kmax_pour(dims->colonnes[j], n_codes);
    }
    const bool interne = delta_interne(n_delta, n_codes);
    if (interne) {  // partial sums only: no block entries in the workspace
        pm.ech = 0;
        pm.partiels = morceaux;
        pm.pas = pas_tache_interne(Rm, Cm);
    }
    pm.act = act;  // the down jobs' x: the experts' SwiGLU rows
    pm.biais = biais;
    const Taches t_delta = par_moe(pm, trc::TACHES_MOE_DELTA, 0), t_gu = par_moe(pm, trc::TACHES_MOE_GU, 0),
                 t_bas = par_moe(pm, trc::TACHES_MOE_BAS, 0), t_gu_topk = par_moe(pm, trc::TACHES_MOE_GU, OPT_TOPK);
    const hipStream_t f = flux_de(flux);
    auto ctl = reinterpret_cast<uint32_t*>(controle.adresse);
    const uint32_t* l = reinterpret_cast<const uint32_t*>(luts.adresse);
    if (norme.adresse != 0) {
        TRC_VERIFIER(norme.octets >= 4ull * C, "norme trop courte");
        TRC_VERIFIER(residu.adresse % 16 == 0 && residu.adresse != x.adresse, "residu non aligne ou confondu avec x");
        TRC_LANCER(fusion_routeur_norme, dim3((experts + 7) / 8), dim3(256), f,
                   reinterpret_cast<const uint16_t*>(routeur.adresse), reinterpret_cast<const float*>(residu.adresse),
                   reinterpret_cast<const float*>(norme.adresse), eps, reinterpret_cast<float*>(x.adresse),
                   reinterpret_cast<const float*>(routeur_biais.adresse), reinterpret_cast<float*>(logits), experts, C);
    } else {
        TRC_LANCER(fusion_routeur, dim3((experts + 7) / 8), dim3(256), f,
                   reinterpret_cast<const uint16_t*>(routeur.adresse), reinterpret_cast<const float*>(x.adresse),
                   reinterpret_cast<const float*>(routeur_biais.adresse), reinterpret_cast<float*>(logits), experts, C);
    }
    if (interne) {
        // four launches: router, gate/up (top-k, DELTA and CODES), down (the SwiGLU rows of its
        // expert, DELTA and CODES), combine; with down blocks under 1024 threads, or a block's share
        // of bias rows past its threads, the k SwiGLU rows are finished once per expert by their own
        // launch between gate/up and down
        const FormeGemv fgu = forme_gemv(R, C, n_codes, 2 * k), fb = forme_gemv(D, R, n_codes, k);
        // bias copies when every block's share of rows fits its threads
        const bool copies = fb.bloc.x == 1024 && (R + fgu.grille.x - 1) / fgu.grille.x <= fgu.bloc.x &&
                            (D + fb.grille.x - 1) / fb.grille.x <= fb.bloc.x && pm.kmax[2] == 2u;
        if (copies) {
            const Taches gu_c = par_moe(pm, trc::TACHES_MOE_GU, OPT_TOPK | OPT_BIAIS),
                         bas_c = par_moe(pm, trc::TACHES_MOE_BAS, OPT_BIAIS);
            if (fgu.bloc.x == 1024)
                TRC_LANCER_N("fusion_codes/gate_up", fusion_codes_gu, fgu.grille, fgu.bloc, f, gu_c, l, ctl);
            else
                TRC_LANCER_CODES("fusion_codes/gate_up", fgu, f, gu_c, l, ctl);
            TRC_LANCER_N("fusion_codes/down", fusion_codes_swiglu, fb.grille, fb.bloc, f, bas_c, l, ctl);
            TRC_LANCER(fusion_finir_combiner, dim3((D + 255) / 256), dim3(256), f, bas_c);
            return TRC_OK;
        }
        TRC_LANCER_CODES("fusion_codes/gate_up", fgu, f, t_gu_topk, l, ctl);
        TRC_LANCER(fusion_finir_swiglu, dim3((R + 255) / 256, k), dim3(256), f, t_gu, reinterpret_cast<float*>(act), R);
        TRC_LANCER_CODES("fusion_codes/down", fb, f, t_bas, l, ctl);
        TRC_LANCER(fusion_finir_combiner, dim3((D + 255) / 256), dim3(256), f, t_bas);
        return TRC_OK;
    }
    TRC_LANCER(fusion_echelles, dim3(grille_echelles(uint64_t(R) * (C / 32), n_delta, 3 * k), 3 * k),
               dim3(trc::FILS_ECHELLES_FUSION), f, t_delta, l, ctl);
    TRC_LANCER_N("fusion_gemv/gate_up", fusion_gemv, forme_gemv(R, C, n_codes, 2 * k).grille,
                 forme_gemv(R, C, n_codes, 2 * k).bloc, f, t_gu, l, ctl);
    TRC_LANCER(fusion_finir_swiglu, dim3((R + 255) / 256, k), dim3(256), f, t_gu, reinterpret_cast<float*>(act), R);
    TRC_LANCER_N("fusion_gemv/down", fusion_gemv, forme_gemv(D, R, n_codes, k).grille,
                 forme_gemv(D, R, n_codes, k).bloc, f, t_bas, l, ctl);
    TRC_LANCER(fusion_finir_combiner, dim3((D + 255) / 256), dim3(256), f, t_bas);
    return TRC_OK;
}
}  // namespace

extern "C" int trc_couche_moe_fusionnee(trc_vue repertoire, uint32_t experts, trc_vue luts, const trc_dims_expert* dims,
                                        trc_vue routeur, trc_vue routeur_biais, trc_vue x, uint32_t k,
                                        trc_vue residu, trc_vue indices, trc_vue poids, trc_vue controle,
                                        trc_vue travail, uint32_t n_delta, uint32_t n_codes, void* flux) {
    return couche_moe(repertoire, experts, luts, dims, routeur, routeur_biais, x, k, residu, indices, poids, controle,
                      travail, n_delta, n_codes, trc_vue{0, 0}, 0.0f, flux);
}

// ------------------------------------------------------------ the allocation-free MoE layer step
// A file-scope device array stands in for the caller's workspace. In host code `scratch` names a
// host-side stand-in, not device memory: its device address is taken once per device, with that
// device current, by hipGetSymbolAddress, and only that address (adresse_scratch) is used.
namespace {
constexpr uint64_t OCTETS_SCRATCH = 16ull << 20;  // holds a gpt-oss layer step at k <= 4 (N_codes >= 16)
constexpr int CARTES_MAX = 64;
__device__ __align__(256) uint8_t scratch[OCTETS_SCRATCH];
std::mutex verrou_scratch;
void* adresse_scratch[CARTES_MAX] = {};

// The device address of `scratch` on device d, taken once (with d current) and kept.
int resoudre_scratch(int d, void** adresse) {
    if (d < 0 || d >= CARTES_MAX) return usage("carte %d hors des %d que la memoire statique couvre", d, CARTES_MAX);
    std::lock_guard<std::mutex> g(verrou_scratch);
    if (adresse_scratch[d] == nullptr) {
        int courante = -1;
        hipError_t e = hipGetDevice(&courante);
        if (e != hipSuccess) return trc::erreur_hip("hipGetDevice", e);
        if (courante != d && (e = hipSetDevice(d)) != hipSuccess) return trc::erreur_hip("hipSetDevice", e);
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (courante != d) (void)hipSetDevice(courante);
        if (e != hipSuccess) return trc::erreur_hip("hipGetSymbolAddress(scratch)", e);
        if (p == nullptr) return usage("adresse nulle pour la memoire statique de la carte %d", d);
        adresse_scratch[d] = p;
    }
    *adresse = adresse_scratch[d];
    return TRC_OK;
}

// The scratch address on the device of `flux` (the current device if flux is null). Resolved by
// trc_contexte_creer (trc::preparer_scratch) for a context's device, else at this first call.
int scratch_de(void* flux, void** adresse) {
    int d = -1;
    hipDevice_t dh = 0;
    if (flux != nullptr && hipStreamGetDevice(reinterpret_cast<hipStream_t>(flux), &dh) == hipSuccess) {
        d = int(dh);
    } else {
        const hipError_t e = hipGetDevice(&d);
        if (e != hipSuccess) return trc::erreur_hip("hipGetDevice", e);
    }
    return resoudre_scratch(d, adresse);
}
}  // namespace

int trc::preparer_scratch(int carte) {
    void* p = nullptr;
    return resoudre_scratch(carte, &p);
}

extern "C" uint64_t trc_octets_scratch(void) { return OCTETS_SCRATCH; }

// trc_couche_moe_fusionnee with the device's static scratch as its workspace: no allocation.
extern "C" int trc_couche_moe_fusionnee_sans_alloc(trc_vue repertoire, uint32_t experts, trc_vue luts,
                                                   const trc_dims_expert* dims, trc_vue routeur,
                                                   trc_vue routeur_biais, trc_vue x, uint32_t k, trc_vue residu,
                                                   trc_vue indices, trc_vue poids, trc_vue controle, uint32_t n_delta,
                                                   uint32_t n_codes, void* flux) {
    const uint64_t besoin = trc_taille_travail_couche_moe(dims, experts, k, n_codes);
    if (besoin == 0) return usage("forme, top-k ou N refuses");
    if (besoin > OCTETS_SCRATCH)
        return usage("l'etape demande %llu o de travail, la memoire statique en a %llu",
                     (unsigned long long)besoin, (unsigned long long)OCTETS_SCRATCH);
    void* p = nullptr;
    const int r = scratch_de(flux, &p);
    if (r != TRC_OK) return r;
    const trc_vue travail{uint64_t(reinterpret_cast<uintptr_t>(p)), OCTETS_SCRATCH};
    return couche_moe(repertoire, experts, luts, dims, routeur, routeur_biais, x, k, residu, indices, poids, controle,
                      travail, n_delta, n_codes, trc_vue{0, 0}, 0.0f, flux);
}

int trc::lancer_couche_moe_normee(trc_vue repertoire, uint32_t experts, trc_vue luts, const trc_dims_expert* dims,
                                  trc_vue routeur, trc_vue routeur_biais, trc_vue norme, float eps, trc_vue h2,
                                  uint32_t k, trc_vue residu, trc_vue indices, trc_vue poids, trc_vue controle,
                                  trc_vue travail, uint32_t n_delta, uint32_t n_codes, void* flux) {
    TRC_VERIFIER(norme.adresse != 0, "norme absente");
    return couche_moe(repertoire, experts, luts, dims, routeur, routeur_biais, h2, k, residu, indices, poids, controle,
                      travail, n_delta, n_codes, norme, eps, flux);
}
