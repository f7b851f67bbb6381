// passe.hpp — fused launches of passe.hip that only the native decode-step driver issues (no
// reference counterpart, not part of the C-ABI): the values are those of the separate entry points
// they replace, in the same operation order.
#pragma once

#include <cstdint>

#include "../../include/troncons_hip.h"

namespace trc {

// rmsnorm(x, norme) then the q, k and v Q8_0 GEMVs of the normed row (w, biais, y, lignes indexed
// q, k, v); colonnes = the row's length, at most 16384.
int lancer_qkv_q8_0(trc_vue x, trc_vue norme, float eps, uint32_t colonnes, const trc_vue w[3],
                    const trc_vue biais[3], const trc_vue y[3], const uint32_t lignes[3], void* flux);

// rope_yarn over q's and k's heads, then ecrire_kv of the rotated k and of v into slot case_kv
// (head dimension at most 64).
int lancer_rope_yarn_kv(trc_vue q, trc_vue k, trc_vue v, trc_vue cache_k, trc_vue cache_v, uint32_t tetes_q,
                        uint32_t tetes_k, uint32_t position, uint32_t case_kv, const trc_params_rope* p, void* flux);

// residu[r] = residu[r] + (W x + b)[r]: gemv_q8_0 then the unweighted combine of its one output.
int lancer_gemv_q8_0_residu(trc_vue w, trc_vue x, trc_vue biais, trc_vue residu, uint32_t lignes, uint32_t colonnes,
                            void* flux);

}  // namespace trc
