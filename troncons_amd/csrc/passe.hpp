// passe.hpp — fused launches of passe.hip that only the native decode-step driver issues (no
// reference counterpart, not part of the C-ABI): the values are those of the separate entry points
// they replace, in the same operation order.
#pragma once

#include <cstdint>

#include "../../include/troncons_hip.h"

namespace trc {

// The rotation coefficients (c, s) in f64 of the 32 pairs of a 64-wide head at `position`
// (rope_yarn's): table = f64[32][2].
int lancer_table_rope(const trc_params_rope* p, uint32_t position, trc_vue table, void* flux);

// rmsnorm(x, norme), the q, k and v Q8_0 GEMVs of the normed row (w, biais, y, lignes indexed q,
// k, v; heads of 64 rows, v as many rows as k), rope_yarn of q and k with the position's table,
// then ecrire_kv of the rotated k and of v into slot case_kv; colonnes = the row's length, at most
// 16384.
int lancer_qkv_q8_0(trc_vue x, trc_vue norme, float eps, uint32_t colonnes, const trc_vue w[3],
                    const trc_vue biais[3], const trc_vue y[3], const uint32_t lignes[3], trc_vue cache_k,
                    trc_vue cache_v, trc_vue table, uint32_t case_kv, void* flux);

// residu[r] = residu[r] + (W x + b)[r]: gemv_q8_0 then the unweighted combine of its one output.
int lancer_gemv_q8_0_residu(trc_vue w, trc_vue x, trc_vue biais, trc_vue residu, uint32_t lignes, uint32_t colonnes,
                            void* flux);

// (fusion.hip) trc_couche_moe_fusionnee over RMSNorm(residu) with `norme`: the router launch
// takes the norm (the rmsnorm kernel's bits) and leaves it in h2, which the later passes read as
// their x; residu then receives the combine. The post-attention norm and the MoE half in one.
int lancer_couche_moe_normee(trc_vue repertoire, uint32_t experts, trc_vue luts, const trc_dims_expert* dims,
                             trc_vue routeur, trc_vue routeur_biais, trc_vue norme, float eps, trc_vue h2, uint32_t k,
                             trc_vue residu, trc_vue indices, trc_vue poids, trc_vue controle, trc_vue travail,
                             uint32_t n_delta, uint32_t n_codes, void* flux);

}  // namespace trc
