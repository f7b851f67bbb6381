// passe.hip — the rest of a gpt-oss layer step around the expert path, for gfx950: the Q8_0 GEMV
// (attention projections, output head) and row (embedding), RMSNorm, the YaRN rotation, the f16
// KV-cache write, decode attention with per-head sinks, argmax. Same names, arguments and results
// as the reference's kernels (moteur/crates/trc-noyaux/noyaux/passe.cuh). The Q8_0 GEMV, the norm
// and the KV write keep the reference's operation order, so their results are bit-identical: the
// Q8_0 GEMV runs one reference "warp" per 32-lane half with the reference's lane order and
// butterfly, the single-vector operations keep their f64 arithmetic and fixed reduction trees. The
// YaRN frequencies and the attention are computed in forms of their own (f64 closed form; a
// one-pass running softmax), equal to the reference's within rounding.
//
// Determinism: no atomics; every reduction follows a tree that depends on sizes only.
#include <hip/hip_runtime.h>

#include <cmath>

#include "commun.hpp"
#include "erreurs.hpp"
#include "norme.hpp"
#include "passe.hpp"

namespace trc {

constexpr uint32_t Q8_OCTETS_BLOC = 34;  // f16 d, then 32 x i8 (ggml Q8_0)
constexpr uint32_t FILS_PASSE = 256;
static_assert(FILS_PASSE == FILS_NORME, "rmsnorm and the Q/K/V launch run the norm with its block size");
constexpr uint32_t FILS_ARGMAX = 1024;
constexpr uint32_t ATTENTION_DIM = 64;
constexpr uint32_t ATTENTION_POSITIONS_MAX = TRC_ATTENTION_POSITIONS_MAX;
constexpr uint32_t QKV_COLONNES_MAX = 16384;  // the normed row lives in LDS (64 KiB)

// The three projections of qkv_q8_0 (q, k, v in that order).
struct Q8Projections {
    const uint8_t* w[3];
    const float* biais[3];
    float* y[3];
    uint32_t lignes[3];
};

__device__ __forceinline__ float f16_vers_f32(uint32_t bits) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
}
__device__ __forceinline__ uint16_t f32_vers_f16(float f) {  // round to nearest even
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Best of two (value, index): larger value, then lower index; a NaN is never better.
__device__ __forceinline__ bool meilleur(float va, uint32_t ia, float vb, uint32_t ib) {
    return va > vb || (va == vb && ia < ib);
}

// YaRN (Peng et al., "YaRN: Efficient Context Window Extension of Large Language Models", 2023),
// with the parameters of gpt-oss's published configuration (passe.cuh:145-167 defines the same
// function): pair i of a d-dim head turns at theta_i = base^(-2i/d). Past the original context
// (facteur s > 1), a pair keeps theta_i if its wavelength is short, takes theta_i / s if it is long,
// and blends linearly in between: theta_i * (1 - g + g / s), g = clamp((i - lo) / (hi - lo), 0, 1),
// where lo and hi are the pair indices whose wavelength 2 pi / theta equals ctx_origine / beta for
// beta = beta_rapide and beta_lent. Variant 1 (llama.cpp) rounds lo down and hi up into [0, d - 1].
// The attention concentration is 1 + 0.1 ln s. All in f64.
__device__ inline double indice_longueur_onde(const trc_params_rope& p, double beta) {
    constexpr double DEUX_PI = 2.0 * 3.14159265358979323846;
    return 0.5 * double(p.dim_tete) * log(p.ctx_origine / (DEUX_PI * beta)) / log(p.base);
}

__device__ inline double inv_freq_yarn(const trc_params_rope& p, uint32_t i, double& concentration) {
    const double theta = exp(-log(p.base) * double(2u * i) / double(p.dim_tete));
    if (p.facteur <= 1.0) {
        concentration = 1.0;
        return theta;
    }
    concentration = 1.0 + 0.1 * log(p.facteur);
    double lo = indice_longueur_onde(p, p.beta_rapide), hi = indice_longueur_onde(p, p.beta_lent);
    if (p.variante == 1u) {
        lo = fmax(floor(lo), 0.0);
        hi = fmin(ceil(hi), double(p.dim_tete - 1u));
    }
    const double g = fmin(fmax((double(i) - lo) / (hi - lo), 0.0), 1.0);
    return theta * ((1.0 - g) + g / p.facteur);
}

}  // namespace trc

// y = W x (+ b), W Q8_0 (passe.cuh:52-97, 213-222): row r is taken by one half-wavefront, lane l
// of which takes blocks b = l, l + 32, ...; in a block s = sum of q_i x_i (one fmaf chain in
// element order), then acc = fmaf(d, s, acc) in increasing b; butterfly over the half. A
// half-wavefront takes LIGNES consecutive rows (the reference's warp takes four; the result of a
// row does not depend on it), and each lane issues the loads of DEPLI of its blocks before using
// them. A block (34 bytes, even address) is read as the 4-byte aligned window that holds it
// (d at byte 0 or 2 of the window, the codes after it): eight dwords and two halves, realigned by a
// 64-bit shift. The half-wavefront's rows are r0 .. r0 + LIGNES - 1; lane 0 hands each row's sum
// (bias not added) to `ecrire(r, s)`. x may be in LDS or global memory.
namespace trc {
template <uint32_t LIGNES, uint32_t DEPLI, class Ecrire>
__device__ __forceinline__ void gemv_q8_0_rangees(const uint8_t* __restrict__ W, const float* __restrict__ x,
                                                  uint32_t R, uint32_t C, uint32_t r0, Ecrire ecrire) {
    const uint32_t voie = threadIdx.x & 31u;
    if (r0 >= R) return;
    const uint32_t B = C / 32u;
    const uint64_t octets_ligne = uint64_t(B) * Q8_OCTETS_BLOC;
    const uintptr_t fin_matrice = reinterpret_cast<uintptr_t>(W) + uint64_t(R) * octets_ligne;
    const f32x4* x4 = reinterpret_cast<const f32x4*>(x);  // x may be in LDS: a generic pointer
    float acc[LIGNES];
    uintptr_t lig[LIGNES];
#pragma unroll
    for (uint32_t i = 0; i < LIGNES; ++i) {
        acc[i] = 0.0f;
        lig[i] = reinterpret_cast<uintptr_t>(W) + uint64_t(min(r0 + i, R - 1u)) * octets_ligne;
    }
    for (uint32_t b0 = voie; b0 < B; b0 += 32u * DEPLI) {
        uint32_t w[DEPLI][LIGNES][9];
        uint32_t decal[DEPLI][LIGNES];
#pragma unroll
        for (uint32_t it = 0; it < DEPLI; ++it) {
            // past the row's end the lane reads its last block again and leaves it unused
            const uint32_t b = min(b0 + 32u * it, B - 1u);
#pragma unroll
            for (uint32_t i = 0; i < LIGNES; ++i) {
                // absolute addresses: W is only 2-byte aligned; a window starting 2 bytes before W
                // stays in W's 4-byte word, hence in its page
                const uintptr_t a = lig[i] + uint64_t(b) * Q8_OCTETS_BLOC;
                const uintptr_t a4 = a & ~uintptr_t(3);
                decal[it][i] = uint32_t(a - a4);  // 0 or 2: where d starts in the window
                const gptr<uint32_t> fen = glob<uint32_t>(reinterpret_cast<const void*>(a4));
#pragma unroll
                for (uint32_t t = 0; t < 8; ++t) w[it][i][t] = fen[t];
                // dword 8 holds the last codes, read as two halves: the high one lies past the block
                // when d sits at byte 0 and is then unused, so its address is clamped to the matrix
                // (no branch around a load, so no load waits for another)
                const gptr<uint16_t> h8 = glob<uint16_t>(reinterpret_cast<const void*>(a4 + 32u));
                const gptr<uint16_t> h9 = glob<uint16_t>(reinterpret_cast<const void*>(min(a4 + 34u, fin_matrice - 2u)));
                w[it][i][8] = uint32_t(h8[0]) | (uint32_t(h9[0]) << 16);
            }
        }
#pragma unroll
        for (uint32_t it = 0; it < DEPLI; ++it) {
            const uint32_t b = b0 + 32u * it;
            if (b >= B) break;
            float xv[32];
#pragma unroll
            for (uint32_t k = 0; k < 8; ++k) {
                const f32x4 t = x4[b * 8u + k];
                xv[4 * k] = t.x;
                xv[4 * k + 1] = t.y;
                xv[4 * k + 2] = t.z;
                xv[4 * k + 3] = t.w;
            }
#pragma unroll
            for (uint32_t i = 0; i < LIGNES; ++i) {
                const uint32_t* wi = w[it][i];
                const float d = f16_vers_f32(decal[it][i] ? (wi[0] >> 16) : (wi[0] & 0xFFFFu));
                // the 32 codes start at byte 2 + decal of the window: realign dwords by 16 or 32 bits
                const uint32_t bits = 8u * (2u + decal[it][i]);
                float s = 0.0f;
#pragma unroll
                for (uint32_t t = 0; t < 8; ++t) {
                    const uint64_t paire = (uint64_t(wi[t + 1]) << 32) | wi[t];
                    const uint32_t q4 = uint32_t(paire >> bits);
#pragma unroll
                    for (uint32_t u = 0; u < 4; ++u)
                        s = fmaf(float(int32_t(q4 << (24u - 8u * u)) >> 24), xv[4 * t + u], s);
                }
                acc[i] = fmaf(d, s, acc[i]);
            }
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < LIGNES; ++i) {
        const float s = somme_demi_f32(acc[i]);
        if (voie == 0 && r0 + i < R) ecrire(r0 + i, s);
    }
}

// Rows of a launch per block.
template <uint32_t LIGNES>
constexpr uint32_t lignes_bloc() {
    return FILS_PASSE / 32u * LIGNES;
}

// x (C floats, C a multiple of 32) copied into the block's LDS with 16-byte loads.
__device__ __forceinline__ void x_vers_lds(const float* __restrict__ x, f32x4* xs, uint32_t C) {
    const gptr<f32x4> x4 = glob<f32x4>(x);
    for (uint32_t j = threadIdx.x; j < C / 4u; j += FILS_PASSE) xs[j] = x4[j];
    __syncthreads();
}

}  // namespace trc

// One launch of y = W x (+ b). gemv_q8_0: four rows per half-wavefront, x read from global memory
// (large matrices: the output head streams its weights with many waves resident);
// gemv_q8_0_court: one row per half-wavefront, x staged in LDS when it fits (C <= QKV_COLONNES_MAX)
// and four of a lane's blocks' loads in flight (small matrices, where a launch has few blocks and
// each wave's chain of loads sets the time).
extern "C" __global__ void __launch_bounds__(trc::FILS_PASSE)
gemv_q8_0(const uint8_t* __restrict__ W, const float* __restrict__ x, const float* __restrict__ biais,
          float* __restrict__ y, float* __restrict__ residu, uint32_t R, uint32_t C) {
    using namespace trc;
    // the same rows, blocks and operation order as gemv_q8_0_rangees, with each row's window
    // loaded right before its use (fewer registers, more waves resident to stream the matrix)
    const uint32_t voie = threadIdx.x & 31u;
    const uint32_t r0 = (blockIdx.x * (FILS_PASSE / 32u) + (threadIdx.x >> 5)) * 4u;
    if (r0 >= R) return;
    const uint32_t B = C / 32u;
    const uint64_t octets_ligne = uint64_t(B) * Q8_OCTETS_BLOC;
    const uintptr_t fin_matrice = reinterpret_cast<uintptr_t>(W) + uint64_t(R) * octets_ligne;
    const gptr<f32x4> x4 = glob<f32x4>(x);
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    uint32_t lig[4];
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) lig[i] = min(r0 + i, R - 1u);
    for (uint32_t b = voie; b < B; b += 32u) {
        float xv[32];
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) {
            const f32x4 t = x4[b * 8u + k];
            xv[4 * k] = t.x;
            xv[4 * k + 1] = t.y;
            xv[4 * k + 2] = t.z;
            xv[4 * k + 3] = t.w;
        }
#pragma unroll
        for (uint32_t i = 0; i < 4; ++i) {
            const uintptr_t a = reinterpret_cast<uintptr_t>(W) + uint64_t(lig[i]) * octets_ligne +
                                uint64_t(b) * Q8_OCTETS_BLOC;
            const uintptr_t a4 = a & ~uintptr_t(3);
            const uint32_t decal = uint32_t(a - a4);
            const gptr<uint32_t> fen = glob<uint32_t>(reinterpret_cast<const void*>(a4));
            uint32_t w[9];
#pragma unroll
            for (uint32_t t = 0; t < 8; ++t) w[t] = fen[t];
            // dword 8 as two halves: the high one lies past the block when d sits at byte 0 and is
            // then unused, so its address is clamped to the matrix (no branch around a load)
            const gptr<uint16_t> h8 = glob<uint16_t>(reinterpret_cast<const void*>(a4 + 32u));
            const gptr<uint16_t> h9 = glob<uint16_t>(reinterpret_cast<const void*>(min(a4 + 34u, fin_matrice - 2u)));
            w[8] = uint32_t(h8[0]) | (uint32_t(h9[0]) << 16);
            const float d = f16_vers_f32(decal ? (w[0] >> 16) : (w[0] & 0xFFFFu));
            const uint32_t bits = 8u * (2u + decal);
            float s = 0.0f;
#pragma unroll
            for (uint32_t t = 0; t < 8; ++t) {
                const uint64_t paire = (uint64_t(w[t + 1]) << 32) | w[t];
                const uint32_t q4 = uint32_t(paire >> bits);
#pragma unroll
                for (uint32_t u = 0; u < 4; ++u)
                    s = fmaf(float(int32_t(q4 << (24u - 8u * u)) >> 24), xv[4 * t + u], s);
            }
            acc[i] = fmaf(d, s, acc[i]);
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < 4; ++i) {
        const float s = somme_demi_f32(acc[i]);
        if (voie == 0 && r0 + i < R) {
            const float v = biais != nullptr ? s + biais[r0 + i] : s;
            if (residu != nullptr)
                residu[r0 + i] = residu[r0 + i] + v;
            else
                y[r0 + i] = v;
        }
    }
}

extern "C" __global__ void __launch_bounds__(trc::FILS_PASSE)
gemv_q8_0_court(const uint8_t* __restrict__ W, const float* __restrict__ x, const float* __restrict__ biais,
                float* __restrict__ y, float* __restrict__ residu, uint32_t R, uint32_t C) {
    using namespace trc;
    extern __shared__ f32x4 xs[];
    // y = W x + b, or with `residu`, residu[r] = residu[r] + (W x + b)[r] (the unweighted combine
    // of one output) instead of storing y
    auto ecrire = [&](uint32_t r, float s) {
        const float v = biais != nullptr ? s + biais[r] : s;
        if (residu != nullptr)
            residu[r] = residu[r] + v;
        else
            y[r] = v;
    };
    const uint32_t r0 = blockIdx.x * lignes_bloc<1>() + (threadIdx.x >> 5);
    if (C <= QKV_COLONNES_MAX) {
        x_vers_lds(x, xs, C);
        gemv_q8_0_rangees<1, 4>(W, reinterpret_cast<const float*>(xs), R, C, r0, ecrire);
    } else {
        gemv_q8_0_rangees<1, 4>(W, x, R, C, r0, ecrire);
    }
}

namespace trc {
// YaRN rotation (NEOX halves) of pair i < d/2 of head xh, in place: o1 = x1 c - x2 s,
// o2 = x2 c + x1 s, c and s the cosine and sine of position * inv_freq_i times the concentration,
// all in f64 (passe.cuh:261-284).
// The pair's coefficients: c and s times the concentration, in f64.
__device__ __forceinline__ void coefficients_paire(uint32_t i, uint32_t position, const trc_params_rope& p, double& c,
                                                   double& s) {
    double m;
    const double inv = inv_freq_yarn(p, i, m);
    sincos(double(position) * inv, &s, &c);
    c *= m;
    s *= m;
}
__device__ __forceinline__ void rotation_paire(float x1, float x2, double c, double s, float& o1, float& o2) {
    const double a = x1, b = x2;
    o1 = float(a * c - b * s);
    o2 = float(b * c + a * s);
}
__device__ __forceinline__ void tourner_paire(float* xh, uint32_t i, uint32_t position, const trc_params_rope& p,
                                              float& o1, float& o2) {
    const uint32_t demi = p.dim_tete / 2u;
    double c, sn;
    coefficients_paire(i, position, p, c, sn);
    rotation_paire(xh[i], xh[i + demi], c, sn, o1, o2);
    xh[i] = o1;
    xh[i + demi] = o2;
}
}  // namespace trc

// The rotation coefficients of one position, (c, s) for pairs 0 .. d/2 - 1 (the same for every
// layer: computed once per position by the decode-step driver).
extern "C" __global__ void __launch_bounds__(64)
table_rope(trc_params_rope p, uint32_t position, double* __restrict__ table) {
    const uint32_t i = threadIdx.x;
    if (i >= p.dim_tete / 2u) return;
    double c, s;
    trc::coefficients_paire(i, position, p, c, s);
    table[2u * i] = c;
    table[2u * i + 1u] = s;
}

// The attention projections of one layer in one launch, with the YaRN rotation and the KV write:
// each block takes the RMSNorm of x with `norme` into LDS (the same values as rmsnorm), then
//  - q or k (heads of 64 rows): block b of head h takes the four row pairs (i, i + 32),
//    i = 4b .. 4b + 3, one row per half-wavefront; the eight values (bias added) meet in LDS and
//    four threads rotate the pairs with the position's coefficients (table_rope: rope_yarn's
//    arithmetic) into y, and for k also into the cache slot, rounded to f16 (ecrire_kv);
//  - v: eight consecutive rows into y and, rounded to f16, into the cache slot.
// The values are those of rmsnorm, three gemv_q8_0, rope_yarn and ecrire_kv.
extern "C" __global__ void __launch_bounds__(trc::FILS_PASSE)
qkv_q8_0(const float* __restrict__ x, const float* __restrict__ norme, float eps, uint32_t C, trc::Q8Projections m,
         uint16_t* __restrict__ cache_k, uint16_t* __restrict__ cache_v, const double* __restrict__ table,
         uint32_t case_kv) {
    using namespace trc;
    extern __shared__ f32x4 hh4[];
    __shared__ double part[FILS_PASSE];
    __shared__ double total;
    __shared__ float paires[8];
    float* hh = reinterpret_cast<float*>(hh4);
    norme_ligne(x, norme, hh, C, eps, part, &total);
    __syncthreads();
    const uint32_t hw = threadIdx.x >> 5;  // half-wavefront 0..7
    const uint32_t nbq = m.lignes[0] / 8u, nbk = m.lignes[1] / 8u, dkv = m.lignes[1];
    uint32_t bloc = blockIdx.x;
    if (bloc < nbq + nbk) {
        const uint32_t j = bloc < nbq ? 0u : 1u;
        if (j == 1u) bloc -= nbq;
        const uint32_t h = bloc / 8u, b = bloc % 8u;
        const float* bj = m.biais[j];
        gemv_q8_0_rangees<1, 4>(m.w[j], hh, m.lignes[j], C, h * 64u + 32u * (hw >> 2) + 4u * b + (hw & 3u),
                                [&](uint32_t r, float s) { paires[hw] = bj != nullptr ? s + bj[r] : s; });
        __syncthreads();
        if (threadIdx.x < 4u) {
            const uint32_t i = 4u * b + threadIdx.x;
            float o1, o2;
            rotation_paire(paires[threadIdx.x], paires[threadIdx.x + 4u], table[2u * i], table[2u * i + 1u], o1, o2);
            float* yh = m.y[j] + uint64_t(h) * 64u;
            yh[i] = o1;
            yh[i + 32u] = o2;
            if (j == 1u) {
                const uint64_t base = uint64_t(case_kv) * dkv + uint64_t(h) * 64u;
                cache_k[base + i] = f32_vers_f16(o1);
                cache_k[base + i + 32u] = f32_vers_f16(o2);
            }
        }
    } else {
        bloc -= nbq + nbk;
        const float* bv = m.biais[2];
        float* yv = m.y[2];
        gemv_q8_0_rangees<1, 4>(m.w[2], hh, m.lignes[2], C, bloc * 8u + hw, [&](uint32_t r, float s) {
            const float v = bv != nullptr ? s + bv[r] : s;
            yv[r] = v;
            cache_v[uint64_t(case_kv) * dkv + r] = f32_vers_f16(v);
        });
    }
}

// Row `ligne` of a Q8_0 matrix -> f32, exact (d has 11 significant bits, q 7: passe.cuh:627-637).
extern "C" __global__ void __launch_bounds__(trc::FILS_PASSE)
ligne_q8_0(const uint8_t* __restrict__ W, uint32_t ligne, uint32_t C, float* __restrict__ y) {
    using namespace trc;
    const uint32_t i = blockIdx.x * FILS_PASSE + threadIdx.x;
    if (i >= C) return;
    const uint8_t* b = W + uint64_t(ligne) * (C / 32u) * Q8_OCTETS_BLOC + uint64_t(i / 32u) * Q8_OCTETS_BLOC;
    const float d = f16_vers_f32(uint32_t(b[0]) | (uint32_t(b[1]) << 8));
    y[i] = d * float(int8_t(b[2 + (i & 31u)]));
}

// RMSNorm of one row per block (passe.cuh:235-259; the arithmetic is norme_ligne's).
extern "C" __global__ void __launch_bounds__(trc::FILS_PASSE)
rmsnorm(const float* __restrict__ x, const float* __restrict__ w, float* y, uint32_t n, float eps) {
    __shared__ double part[trc::FILS_PASSE];
    __shared__ double total;
    trc::norme_ligne(x + uint64_t(blockIdx.x) * n, w, y + uint64_t(blockIdx.x) * n, n, eps, part, &total);
}


// YaRN rotation of one head per block, in place; heads 0 .. tetes_q - 1 are q's, then k's.
extern "C" __global__ void __launch_bounds__(64)
rope_yarn(float* __restrict__ q, float* __restrict__ k, uint32_t tetes_q, uint32_t tetes_k, uint32_t position,
          trc_params_rope p) {
    const uint32_t i = threadIdx.x;
    if (i >= p.dim_tete / 2u || blockIdx.x >= tetes_q + tetes_k) return;
    float* xh = blockIdx.x < tetes_q ? q + uint64_t(blockIdx.x) * p.dim_tete
                                     : k + uint64_t(blockIdx.x - tetes_q) * p.dim_tete;
    float o1, o2;
    trc::tourner_paire(xh, i, position, p, o1, o2);
}

// k and v rounded to f16 (nearest even) into slot case_kv of the caches (passe.cuh:286-296).
extern "C" __global__ void __launch_bounds__(trc::FILS_PASSE)
ecrire_kv(const float* __restrict__ k, const float* __restrict__ v, uint16_t* __restrict__ cache_k,
          uint16_t* __restrict__ cache_v, uint32_t dkv, uint32_t case_kv) {
    const uint32_t i = blockIdx.x * trc::FILS_PASSE + threadIdx.x;
    if (i >= dkv) return;
    const uint64_t o = uint64_t(case_kv) * dkv + i;
    cache_k[o] = trc::f32_vers_f16(k[i]);
    cache_v[o] = trc::f32_vers_f16(v[i]);
}

// Decode attention of one position for query head h (the result of passe.cuh:298-373, within
// float rounding): scores s_j = (q . k_j) * scale over the positions j in [debut, fin) (slot
// j mod anneau in a windowed layer), then out = sum_j exp(s_j - M) v_j / (sum_j exp(s_j - M) +
// exp(sink - M)), M the largest of the scores and the sink. Query head h reads kv head
// h / (heads / kv heads).
//
// One pass with a running softmax (Milakov & Gimelshein, "Online normalizer calculation for
// softmax", 2018): the block's four wavefronts take chunks of 64 positions in turn (chunk c to
// wavefront c mod 4). In a chunk, lane p scores position 64c + p; the wavefront's running maximum
// moves to include the chunk's, and its running sum and its 64 running outputs (lane = dimension)
// are rescaled by exp(old max - new max) before the chunk's terms are added; each position's weight
// reaches the 64 dimensions through the wavefront's 64 LDS words. The four (max, sum, outputs) are
// merged with the sink at the end, in wavefront order. No score array: any number of positions
// fits in the block's 2 KiB of LDS. The caches hold f16 (attention) or f32 (attention_kvf32).
namespace trc {
__device__ __forceinline__ float lire_kv(uint16_t b) { return f16_vers_f32(b); }
__device__ __forceinline__ float lire_kv(float v) { return v; }

// q . k for one stored key row of 64 values, q in LDS as 16 float4: four interleaved partial
// chains (dimensions 4u + 0..3 of each group of 16) added pairwise at the end.
__device__ __forceinline__ float produit_cle(const f32x4* qs, const uint16_t* kr) {
    const gptr<u32x4> k4 = glob<u32x4>(kr);
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t b = 0; b < 8; ++b) {
        const u32x4 w = k4[b];
        const f32x4 qa = qs[2 * b], qb = qs[2 * b + 1];
        a[0] = fmaf(qa.x, f16_vers_f32(w.x & 0xFFFFu), a[0]);
        a[1] = fmaf(qa.y, f16_vers_f32(w.x >> 16), a[1]);
        a[2] = fmaf(qa.z, f16_vers_f32(w.y & 0xFFFFu), a[2]);
        a[3] = fmaf(qa.w, f16_vers_f32(w.y >> 16), a[3]);
        a[0] = fmaf(qb.x, f16_vers_f32(w.z & 0xFFFFu), a[0]);
        a[1] = fmaf(qb.y, f16_vers_f32(w.z >> 16), a[1]);
        a[2] = fmaf(qb.z, f16_vers_f32(w.w & 0xFFFFu), a[2]);
        a[3] = fmaf(qb.w, f16_vers_f32(w.w >> 16), a[3]);
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}
__device__ __forceinline__ float produit_cle(const f32x4* qs, const float* kr) {
    const gptr<f32x4> k4 = glob<f32x4>(kr);
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t b = 0; b < 16; ++b) {
        const f32x4 w = k4[b], qv = qs[b];
        a[0] = fmaf(qv.x, w.x, a[0]);
        a[1] = fmaf(qv.y, w.y, a[1]);
        a[2] = fmaf(qv.z, w.z, a[2]);
        a[3] = fmaf(qv.w, w.w, a[3]);
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

__device__ __forceinline__ float max_vague(float v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = fmaxf(v, __shfl_xor(v, d));
    return v;
}
__device__ __forceinline__ float somme_vague(float v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d);
    return v;
}

template <typename T>
__device__ __forceinline__ void attention_tete(const float* __restrict__ q, const T* __restrict__ cache_k,
                                               const T* __restrict__ cache_v, const float* __restrict__ puits,
                                               float* __restrict__ sortie, const trc_params_attention& p) {
    constexpr uint32_t VAGUES = FILS_PASSE / 64u;
    __shared__ f32x4 qs[ATTENTION_DIM / 4];
    __shared__ float poids[VAGUES][64];
    __shared__ float sorties[VAGUES][ATTENTION_DIM];
    __shared__ float maxima[VAGUES], sommes[VAGUES];
    const uint32_t t = threadIdx.x, w = t >> 6, lane = t & 63u;
    const uint32_t h = blockIdx.x;
    const uint32_t hk = h / (p.tetes / p.tetes_kv);
    const uint64_t dkv = uint64_t(p.tetes_kv) * ATTENTION_DIM;
    const uint32_t n = p.fin - p.debut;
    if (t < ATTENTION_DIM / 4u) qs[t] = glob<f32x4>(q + uint64_t(h) * ATTENTION_DIM)[t];
    __syncthreads();

    const T* cles = cache_k + uint64_t(hk) * ATTENTION_DIM;
    const T* valeurs = cache_v + uint64_t(hk) * ATTENTION_DIM + lane;
    float m = -INFINITY, z = 0.0f, o = 0.0f;
    for (uint32_t c0 = 64u * w; c0 < n; c0 += 64u * VAGUES) {
        const uint32_t pos0 = p.debut + c0;
        const uint32_t case0 = p.anneau ? pos0 % p.anneau : pos0;  // slots of the chunk: case0 + k, wrapped
        auto case_de = [&](uint32_t k) {
            const uint32_t c = case0 + k;
            return p.anneau && c >= p.anneau ? c - p.anneau : c;
        };
        const bool ok = c0 + lane < n;
        const float s = ok ? produit_cle(qs, cles + uint64_t(case_de(lane)) * dkv) * p.echelle : -INFINITY;
        const float m2 = fmaxf(m, max_vague(s));
        // While every score so far is -inf (keys with an infinite component), m2 is -inf and
        // exp(-inf - -inf) would be NaN: no term has weight yet, as in the reference, whose maximum
        // includes the sink before any exponential (passe.cuh:306-371).
        const float alpha = m == -INFINITY ? 0.0f : expf(m - m2);  // 0 for the first chunk (m = -inf)
        const float e = m2 == -INFINITY ? 0.0f : expf(s - m2);      // 0 for lanes past the end
        z = fmaf(z, alpha, somme_vague(e));
        poids[w][lane] = e;  // read back by this wavefront only, in program order
        const uint32_t nc = min(64u, n - c0);
        float acc = 0.0f;
        constexpr uint32_t LOT = 8;
        for (uint32_t k0 = 0; k0 < nc; k0 += LOT) {
            T vv[LOT];
#pragma unroll
            for (uint32_t u = 0; u < LOT; ++u) vv[u] = valeurs[uint64_t(case_de(min(k0 + u, nc - 1u))) * dkv];
#pragma unroll
            for (uint32_t u = 0; u < LOT; ++u)
                if (k0 + u < nc) acc = fmaf(poids[w][k0 + u], lire_kv(vv[u]), acc);
        }
        o = fmaf(o, alpha, acc);
        m = m2;
    }
    if (lane == 0) {
        maxima[w] = m;
        sommes[w] = z;
    }
    sorties[w][lane] = o;
    __syncthreads();
    if (t < ATTENTION_DIM) {
        const float puits_h = puits[h];
        float mg = puits_h;
#pragma unroll
        for (uint32_t v = 0; v < VAGUES; ++v) mg = fmaxf(mg, maxima[v]);
        float zg = expf(puits_h - mg), og = 0.0f;
#pragma unroll
        for (uint32_t v = 0; v < VAGUES; ++v) {
            const float f = expf(maxima[v] - mg);
            zg = fmaf(sommes[v], f, zg);
            og = fmaf(sorties[v][t], f, og);
        }
        sortie[uint64_t(h) * ATTENTION_DIM + t] = og / zg;
    }
}
}  // namespace trc

extern "C" __global__ void __launch_bounds__(trc::FILS_PASSE)
attention(const float* __restrict__ q, const uint16_t* __restrict__ cache_k, const uint16_t* __restrict__ cache_v,
          const float* __restrict__ puits, float* __restrict__ sortie, trc_params_attention p) {
    trc::attention_tete(q, cache_k, cache_v, puits, sortie, p);
}

extern "C" __global__ void __launch_bounds__(trc::FILS_PASSE)
attention_kvf32(const float* __restrict__ q, const float* __restrict__ cache_k, const float* __restrict__ cache_v,
                const float* __restrict__ puits, float* __restrict__ sortie, trc_params_attention p) {
    trc::attention_tete(q, cache_k, cache_v, puits, sortie, p);
}

// k and v copied unrounded into slot case_kv of f32 caches (passe.cuh:379-387).
extern "C" __global__ void __launch_bounds__(trc::FILS_PASSE)
ecrire_kv_f32(const float* __restrict__ k, const float* __restrict__ v, float* __restrict__ cache_k,
              float* __restrict__ cache_v, uint32_t dkv, uint32_t case_kv) {
    const uint32_t i = blockIdx.x * trc::FILS_PASSE + threadIdx.x;
    if (i >= dkv) return;
    const uint64_t o = uint64_t(case_kv) * dkv + i;
    cache_k[o] = k[i];
    cache_v[o] = v[i];
}

// Index of the largest of n floats: thread t scans i = t, t + 1024, ..., then a fixed tree; ties go
// to the lower index, NaN is never chosen (passe.cuh:639-666).
extern "C" __global__ void __launch_bounds__(trc::FILS_ARGMAX)
argmax(const float* __restrict__ v, uint32_t n, uint32_t* __restrict__ sortie) {
    using namespace trc;
    __shared__ float pv[FILS_ARGMAX];
    __shared__ uint32_t pi[FILS_ARGMAX];
    const uint32_t t = threadIdx.x;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    auto voir = [&](float xv, uint32_t i) {
        if (meilleur(xv, i, bv, bi)) {
            bv = xv;
            bi = i;
        }
    };
    // The result does not depend on the order the values are seen in: the scalar head up to a
    // 16-byte boundary, then 16-byte loads, four in flight per thread, then the scalar tail.
    const uint32_t tete = min(n, uint32_t((16u - (reinterpret_cast<uintptr_t>(v) & 15u)) & 15u) / 4u);
    for (uint32_t i = t; i < tete; i += FILS_ARGMAX) voir(v[i], i);
    const uint32_t n4 = (n - tete) / 4u;
    const f32x4* v4 = reinterpret_cast<const f32x4*>(v + tete);
    for (uint32_t j0 = t; j0 < n4; j0 += 4u * FILS_ARGMAX) {
        f32x4 c[4];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u)
            if (j0 + u * FILS_ARGMAX < n4) c[u] = v4[j0 + u * FILS_ARGMAX];
#pragma unroll
        for (uint32_t u = 0; u < 4; ++u) {
            const uint32_t j = j0 + u * FILS_ARGMAX;
            if (j < n4) {
                const uint32_t i = tete + 4u * j;
                voir(c[u].x, i);
                voir(c[u].y, i + 1u);
                voir(c[u].z, i + 2u);
                voir(c[u].w, i + 3u);
            }
        }
    }
    for (uint32_t i = tete + 4u * n4 + t; i < n; i += FILS_ARGMAX) voir(v[i], i);
    pv[t] = bv;
    pi[t] = bi;
    __syncthreads();
    for (uint32_t k = FILS_ARGMAX / 2u; k > 0; k >>= 1) {
        if (t < k && meilleur(pv[t + k], pi[t + k], pv[t], pi[t])) {
            pv[t] = pv[t + k];
            pi[t] = pi[t + k];
        }
        __syncthreads();
    }
    if (t == 0) sortie[0] = pi[0];
}

// ============================================================================ C-ABI launch layer
namespace {
inline hipStream_t flux_de(void* f) { return reinterpret_cast<hipStream_t>(f); }

// Below this many rows a GEMV takes one row per half-wavefront (more waves, shorter load chains).
constexpr uint32_t GEMV_COURT_LIGNES = 32768;

void lancer_gemv(const uint8_t* W, const float* x, const float* biais, float* y, float* residu, uint32_t R, uint32_t C,
                 hipStream_t f) {
    if (R < GEMV_COURT_LIGNES) {
        const size_t lds = C <= trc::QKV_COLONNES_MAX ? 4u * size_t(C) : 0u;
        constexpr uint32_t rb = trc::lignes_bloc<1>();
        hipLaunchKernelGGL(gemv_q8_0_court, dim3((R + rb - 1) / rb), dim3(trc::FILS_PASSE), lds, f, W, x, biais, y,
                           residu, R, C);
    } else {
        constexpr uint32_t rb = trc::lignes_bloc<4>();
        hipLaunchKernelGGL(gemv_q8_0, dim3((R + rb - 1) / rb), dim3(trc::FILS_PASSE), 0, f, W, x, biais, y, residu, R,
                           C);
    }
}
}  // namespace

extern "C" int trc_gemv_q8_0(trc_vue w, trc_vue x, trc_vue biais, trc_vue y, uint32_t lignes, uint32_t colonnes,
                             void* flux) {
    TRC_VERIFIER(lignes > 0 && colonnes > 0 && colonnes % 32 == 0, "forme %u x %u", lignes, colonnes);
    const uint64_t octets = uint64_t(lignes) * (colonnes / 32) * trc::Q8_OCTETS_BLOC;
    TRC_VERIFIER(w.adresse != 0 && w.octets >= octets && w.adresse % 2 == 0,
                 "matrice Q8_0 de %llu o, %llu o demandes (adresse paire)", (unsigned long long)w.octets,
                 (unsigned long long)octets);
    TRC_VERIFIER(x.adresse != 0 && x.octets >= 4ull * colonnes && x.adresse % 16 == 0,
                 "x trop court ou non aligne sur 16");
    TRC_VERIFIER(y.adresse != 0 && y.octets >= 4ull * lignes, "y trop court");
    TRC_VERIFIER(biais.adresse == 0 || biais.octets >= 4ull * lignes, "biais trop court");
    lancer_gemv(reinterpret_cast<const uint8_t*>(w.adresse), reinterpret_cast<const float*>(x.adresse),
                reinterpret_cast<const float*>(biais.adresse), reinterpret_cast<float*>(y.adresse), nullptr, lignes,
                colonnes, flux_de(flux));
    return trc::apres_lancement("gemv_q8_0");
}

extern "C" int trc_ligne_q8_0(trc_vue w, uint32_t ligne, uint32_t colonnes, trc_vue y, void* flux) {
    TRC_VERIFIER(colonnes > 0 && colonnes % 32 == 0, "%u colonnes", colonnes);
    const uint64_t ol = uint64_t(colonnes / 32) * trc::Q8_OCTETS_BLOC;
    TRC_VERIFIER(w.adresse != 0 && y.adresse != 0 && w.octets >= (uint64_t(ligne) + 1) * ol &&
                     y.octets >= 4ull * colonnes,
                 "ligne_q8_0 : vues trop courtes");
    hipLaunchKernelGGL(ligne_q8_0, dim3((colonnes + trc::FILS_PASSE - 1) / trc::FILS_PASSE), dim3(trc::FILS_PASSE),
                       0, flux_de(flux), reinterpret_cast<const uint8_t*>(w.adresse), ligne, colonnes,
                       reinterpret_cast<float*>(y.adresse));
    return trc::apres_lancement("ligne_q8_0");
}

extern "C" int trc_rmsnorm(trc_vue x, trc_vue w, trc_vue y, uint32_t n, uint32_t lignes, float eps, void* flux) {
    TRC_VERIFIER(n > 0 && lignes > 0, "rmsnorm de %u x %u", lignes, n);
    const uint64_t o = 4ull * n * lignes;
    TRC_VERIFIER(x.adresse && w.adresse && y.adresse && x.octets >= o && y.octets >= o && w.octets >= 4ull * n,
                 "rmsnorm : vues trop courtes");
    hipLaunchKernelGGL(rmsnorm, dim3(lignes), dim3(trc::FILS_PASSE), 0, flux_de(flux),
                       reinterpret_cast<const float*>(x.adresse), reinterpret_cast<const float*>(w.adresse),
                       reinterpret_cast<float*>(y.adresse), n, eps);
    return trc::apres_lancement("rmsnorm");
}

extern "C" int trc_rope_yarn(trc_vue q, trc_vue k, uint32_t tetes_q, uint32_t tetes_k, uint32_t position,
                             const trc_params_rope* p, void* flux) {
    if (p == nullptr) return trc::usage("parametres de YaRN absents");
    TRC_VERIFIER(p->dim_tete > 0 && p->dim_tete % 2 == 0 && p->dim_tete <= 128, "dimension de tete %u", p->dim_tete);
    TRC_VERIFIER(p->variante <= 1, "variante de YaRN %u", p->variante);
    TRC_VERIFIER(tetes_q + tetes_k > 0, "aucune tete");
    const uint64_t d = p->dim_tete;
    TRC_VERIFIER((tetes_q == 0 || (q.adresse && q.octets >= 4 * d * tetes_q)) &&
                     (tetes_k == 0 || (k.adresse && k.octets >= 4 * d * tetes_k)),
                 "rope : vues trop courtes");
    hipLaunchKernelGGL(rope_yarn, dim3(tetes_q + tetes_k), dim3(64), 0, flux_de(flux),
                       reinterpret_cast<float*>(q.adresse), reinterpret_cast<float*>(k.adresse), tetes_q, tetes_k,
                       position, *p);
    return trc::apres_lancement("rope_yarn");
}

extern "C" int trc_ecrire_kv(trc_vue k, trc_vue v, trc_vue cache_k, trc_vue cache_v, uint32_t dkv, uint32_t case_kv,
                             void* flux) {
    TRC_VERIFIER(dkv > 0, "dkv nul");
    const uint64_t fin = 2ull * (uint64_t(case_kv) + 1) * dkv;
    TRC_VERIFIER(k.adresse && v.adresse && k.octets >= 4ull * dkv && v.octets >= 4ull * dkv, "k ou v trop court");
    TRC_VERIFIER(cache_k.adresse && cache_v.adresse && cache_k.octets >= fin && cache_v.octets >= fin,
                 "case %u hors du cache", case_kv);
    hipLaunchKernelGGL(ecrire_kv, dim3((dkv + trc::FILS_PASSE - 1) / trc::FILS_PASSE), dim3(trc::FILS_PASSE), 0,
                       flux_de(flux), reinterpret_cast<const float*>(k.adresse),
                       reinterpret_cast<const float*>(v.adresse), reinterpret_cast<uint16_t*>(cache_k.adresse),
                       reinterpret_cast<uint16_t*>(cache_v.adresse), dkv, case_kv);
    return trc::apres_lancement("ecrire_kv");
}

namespace {
// Noyaux::attention / attention_kvf32 (lib.rs:366-381, 396-411): the reference's checks, then one
// block per query head; `octets` = bytes per stored value (2 or 4).
int verifier_attention(trc_vue q, trc_vue cache_k, trc_vue cache_v, trc_vue puits, trc_vue sortie,
                       const trc_params_attention* p, uint64_t octets) {
    if (p == nullptr) return trc::usage("parametres d'attention absents");
    TRC_VERIFIER(p->dim_tete == 64 && p->tetes_kv > 0 && p->tetes > 0 && p->tetes % p->tetes_kv == 0,
                 "tetes %u / %u de dimension %u", p->tetes, p->tetes_kv, p->dim_tete);
    TRC_VERIFIER(p->fin >= p->debut && p->fin - p->debut <= trc::ATTENTION_POSITIONS_MAX, "positions [%u, %u)",
                 p->debut, p->fin);
    TRC_VERIFIER(p->anneau == 0 || p->fin - p->debut <= p->anneau, "plus de positions que de cases dans l'anneau");
    const uint64_t cases = p->anneau > 0 ? p->anneau : p->fin;
    const uint64_t dkv = uint64_t(p->tetes_kv) * 64;
    TRC_VERIFIER(cache_k.adresse && cache_v.adresse && cache_k.octets >= octets * cases * dkv &&
                     cache_v.octets >= octets * cases * dkv,
                 "cache trop court");
    TRC_VERIFIER(cache_k.adresse % 16 == 0, "cache des cles non aligne sur 16");
    TRC_VERIFIER(q.adresse && sortie.adresse && puits.adresse && q.octets >= 4ull * 64 * p->tetes &&
                     sortie.octets >= 4ull * 64 * p->tetes && puits.octets >= 4ull * p->tetes,
                 "attention : vues trop courtes");
    return TRC_OK;
}
}  // namespace

extern "C" int trc_attention(trc_vue q, trc_vue cache_k, trc_vue cache_v, trc_vue puits, trc_vue sortie,
                             const trc_params_attention* p, void* flux) {
    const int r = verifier_attention(q, cache_k, cache_v, puits, sortie, p, 2);
    if (r != TRC_OK) return r;
    hipLaunchKernelGGL(attention, dim3(p->tetes), dim3(trc::FILS_PASSE), 0, flux_de(flux),
                       reinterpret_cast<const float*>(q.adresse), reinterpret_cast<const uint16_t*>(cache_k.adresse),
                       reinterpret_cast<const uint16_t*>(cache_v.adresse), reinterpret_cast<const float*>(puits.adresse),
                       reinterpret_cast<float*>(sortie.adresse), *p);
    return trc::apres_lancement("attention");
}

extern "C" int trc_attention_kvf32(trc_vue q, trc_vue cache_k, trc_vue cache_v, trc_vue puits, trc_vue sortie,
                                   const trc_params_attention* p, void* flux) {
    const int r = verifier_attention(q, cache_k, cache_v, puits, sortie, p, 4);
    if (r != TRC_OK) return r;
    hipLaunchKernelGGL(attention_kvf32, dim3(p->tetes), dim3(trc::FILS_PASSE), 0, flux_de(flux), reinterpret_cast<const float*>(q.adresse),
                       reinterpret_cast<const float*>(cache_k.adresse), reinterpret_cast<const float*>(cache_v.adresse),
                       reinterpret_cast<const float*>(puits.adresse), reinterpret_cast<float*>(sortie.adresse), *p);
    return trc::apres_lancement("attention_kvf32");
}

extern "C" int trc_ecrire_kv_f32(trc_vue k, trc_vue v, trc_vue cache_k, trc_vue cache_v, uint32_t dkv,
                                 uint32_t case_kv, void* flux) {
    TRC_VERIFIER(dkv > 0, "dkv nul");
    const uint64_t fin = 4ull * (uint64_t(case_kv) + 1) * dkv;
    TRC_VERIFIER(k.adresse && v.adresse && k.octets >= 4ull * dkv && v.octets >= 4ull * dkv, "k ou v trop court");
    TRC_VERIFIER(cache_k.adresse && cache_v.adresse && cache_k.octets >= fin && cache_v.octets >= fin,
                 "case %u hors du cache f32", case_kv);
    hipLaunchKernelGGL(ecrire_kv_f32, dim3((dkv + trc::FILS_PASSE - 1) / trc::FILS_PASSE), dim3(trc::FILS_PASSE), 0,
                       flux_de(flux), reinterpret_cast<const float*>(k.adresse),
                       reinterpret_cast<const float*>(v.adresse), reinterpret_cast<float*>(cache_k.adresse),
                       reinterpret_cast<float*>(cache_v.adresse), dkv, case_kv);
    return trc::apres_lancement("ecrire_kv_f32");
}

extern "C" int trc_argmax(trc_vue v, uint32_t n, trc_vue sortie, void* flux) {
    TRC_VERIFIER(n > 0 && v.adresse && sortie.adresse && v.octets >= 4ull * n && sortie.octets >= 4,
                 "argmax : vues trop courtes");
    hipLaunchKernelGGL(argmax, dim3(1), dim3(trc::FILS_ARGMAX), 0, flux_de(flux),
                       reinterpret_cast<const float*>(v.adresse), n, reinterpret_cast<uint32_t*>(sortie.adresse));
    return trc::apres_lancement("argmax");
}

// ============================================================================ fused launches of the native driver
// No reference counterpart: the decode-step driver issues these in place of rmsnorm + three
// gemv_q8_0 + rope_yarn + ecrire_kv, and gemv_q8_0 + combiner; the values are the same.
namespace trc {

int lancer_qkv_q8_0(trc_vue x, trc_vue norme, float eps, uint32_t colonnes, const trc_vue w[3],
                    const trc_vue biais[3], const trc_vue y[3], const uint32_t lignes[3], trc_vue cache_k,
                    trc_vue cache_v, trc_vue table, uint32_t case_kv, void* flux) {
    TRC_VERIFIER(colonnes > 0 && colonnes % 32 == 0 && colonnes <= QKV_COLONNES_MAX, "qkv : %u colonnes", colonnes);
    TRC_VERIFIER(x.adresse && norme.adresse && x.octets >= 4ull * colonnes && norme.octets >= 4ull * colonnes,
                 "qkv : x ou norme trop court");
    TRC_VERIFIER(table.adresse && table.adresse % 8 == 0 && table.octets >= 16 * 32, "qkv : table de rotation");
    TRC_VERIFIER(lignes[0] > 0 && lignes[0] % 64 == 0 && lignes[1] > 0 && lignes[1] % 64 == 0 && lignes[2] == lignes[1],
                 "qkv : %u / %u / %u lignes (tetes de 64, v comme k)", lignes[0], lignes[1], lignes[2]);
    const uint64_t fin = 2ull * (uint64_t(case_kv) + 1) * lignes[1];
    TRC_VERIFIER(cache_k.adresse && cache_v.adresse && cache_k.octets >= fin && cache_v.octets >= fin,
                 "qkv : case %u hors du cache", case_kv);
    Q8Projections m;
    uint32_t blocs = 0;
    for (int j = 0; j < 3; ++j) {
        const uint64_t octets = uint64_t(lignes[j]) * (colonnes / 32) * Q8_OCTETS_BLOC;
        TRC_VERIFIER(w[j].adresse && w[j].octets >= octets && w[j].adresse % 2 == 0, "qkv : matrice %d", j);
        TRC_VERIFIER(y[j].adresse && y[j].octets >= 4ull * lignes[j], "qkv : sortie %d trop courte", j);
        TRC_VERIFIER(biais[j].adresse == 0 || biais[j].octets >= 4ull * lignes[j], "qkv : biais %d trop court", j);
        m.w[j] = reinterpret_cast<const uint8_t*>(w[j].adresse);
        m.biais[j] = reinterpret_cast<const float*>(biais[j].adresse);
        m.y[j] = reinterpret_cast<float*>(y[j].adresse);
        m.lignes[j] = lignes[j];
        blocs += lignes[j] / 8;
    }
    hipLaunchKernelGGL(qkv_q8_0, dim3(blocs), dim3(FILS_PASSE), 4u * colonnes, flux_de(flux),
                       reinterpret_cast<const float*>(x.adresse), reinterpret_cast<const float*>(norme.adresse), eps,
                       colonnes, m, reinterpret_cast<uint16_t*>(cache_k.adresse),
                       reinterpret_cast<uint16_t*>(cache_v.adresse), reinterpret_cast<const double*>(table.adresse),
                       case_kv);
    return apres_lancement("qkv_q8_0");
}

int lancer_table_rope(const trc_params_rope* p, uint32_t position, trc_vue table, void* flux) {
    TRC_VERIFIER(p && p->dim_tete == 64 && p->variante <= 1, "table de rotation : tetes de 64 seulement");
    TRC_VERIFIER(table.adresse && table.adresse % 8 == 0 && table.octets >= 16 * 32, "table de rotation trop courte");
    hipLaunchKernelGGL(table_rope, dim3(1), dim3(64), 0, flux_de(flux), *p, position,
                       reinterpret_cast<double*>(table.adresse));
    return apres_lancement("table_rope");
}

int lancer_gemv_q8_0_residu(trc_vue w, trc_vue x, trc_vue biais, trc_vue residu, uint32_t lignes, uint32_t colonnes,
                            void* flux) {
    TRC_VERIFIER(lignes > 0 && colonnes > 0 && colonnes % 32 == 0, "forme %u x %u", lignes, colonnes);
    const uint64_t octets = uint64_t(lignes) * (colonnes / 32) * Q8_OCTETS_BLOC;
    TRC_VERIFIER(w.adresse != 0 && w.octets >= octets && w.adresse % 2 == 0, "matrice Q8_0 trop courte");
    TRC_VERIFIER(x.adresse != 0 && x.octets >= 4ull * colonnes && x.adresse % 16 == 0,
                 "x trop court ou non aligne sur 16");
    TRC_VERIFIER(residu.adresse != 0 && residu.octets >= 4ull * lignes, "residu trop court");
    TRC_VERIFIER(biais.adresse == 0 || biais.octets >= 4ull * lignes, "biais trop court");
    lancer_gemv(reinterpret_cast<const uint8_t*>(w.adresse), reinterpret_cast<const float*>(x.adresse),
                reinterpret_cast<const float*>(biais.adresse), nullptr, reinterpret_cast<float*>(residu.adresse), lignes,
                colonnes, flux_de(flux));
    return apres_lancement("gemv_q8_0");
}

}  // namespace trc
