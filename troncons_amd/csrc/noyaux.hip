// noyaux.hip — the reference kernel API of the expert hot path (Noyaux, moteur/crates/trc-noyaux/
// src/lib.rs), written for gfx950.
//
// Same kernel names, arguments and results as the reference's (decodeur.cuh, gemv.cuh, passe.cuh),
// so that the engine's launch layer maps one to one. The slot decoders run the fused path's rANS
// engine (two tiles per wavefront, LDS word rings, 8-byte LUT entries) with a consumer that stores
// into the slot; the GEMVs produce the reference's bits under the operation-order contract stated
// above them, on a wave64 mapping of their own.
//
// Determinism: no floating-point atomics; the only atomics are integer control counters.
#include <hip/hip_runtime.h>

#include "commun.hpp"
#include "emplacement.hpp"
#include "entiers.hpp"
#include "erreurs.hpp"
#include "fusion_corps.hpp"
#include "selection.hpp"

namespace trc {

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
    __shared__ trc::LdsEchelles<trc::FILS_ECHELLES> s;
    trc::decoder_echelles_corps(partie, emplacement, luts, dims, controle, s);
}

extern "C" __global__ void __launch_bounds__(trc::FILS_CODES_SLOT)
decoder_codes(const uint8_t* __restrict__ partie, uint8_t* __restrict__ emplacement, const uint32_t* __restrict__ luts,
              trc_dims_expert dims, uint32_t* __restrict__ controle) {
    __shared__ trc::LdsCodes s;
    trc::decoder_codes_corps(partie, emplacement, luts, dims, controle, s);
}

extern "C" __global__ void __launch_bounds__(trc::FILS_ECHELLES)
decoder_echelles_lot(const trc::DescDecodage* __restrict__ descs, trc_dims_expert dims) {
    __shared__ trc::LdsEchelles<trc::FILS_ECHELLES> s;
    const trc::DescDecodage d = descs[blockIdx.z];
    trc::decoder_echelles_corps(reinterpret_cast<const uint8_t*>(d.partie), reinterpret_cast<uint8_t*>(d.emplacement),
                                reinterpret_cast<const uint32_t*>(d.luts), dims,
                                reinterpret_cast<uint32_t*>(d.controle), s);
}

extern "C" __global__ void __launch_bounds__(trc::FILS_CODES_SLOT)
decoder_codes_lot(const trc::DescDecodage* __restrict__ descs, trc_dims_expert dims) {
    __shared__ trc::LdsCodes s;
    const trc::DescDecodage d = descs[blockIdx.z];
    trc::decoder_codes_corps(reinterpret_cast<const uint8_t*>(d.partie), reinterpret_cast<uint8_t*>(d.emplacement),
                             reinterpret_cast<const uint32_t*>(d.luts), dims, reinterpret_cast<uint32_t*>(d.controle),
                             s);
}

// Raw-file path (flag bit 2): the slot's three regions — codes (16 bytes per block), scales (one
// byte per block), biases (4 bytes per row) — copied from the CODES_BRUTS, ECHELLES_BRUTES and
// BIAIS streams as one list of 16-byte units over the grid. Sources are 16-byte aligned (streams
// are, in a 16-byte aligned part), destinations 256-byte aligned; a region's last unit, when its
// length is not a multiple of 16, is copied byte by byte, so no byte outside a region is written.
namespace trc {
__device__ __forceinline__ void copier_unite(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint32_t u,
                                             uint32_t octets) {
    const uint32_t o = 16u * u;
    if (o + 16u <= octets) {
        ecrire_global<u32x4>(dst + o, *glob<u32x4>(src + o));
    } else {
        for (uint32_t k = o; k < octets; ++k) dst[k] = glob<uint8_t>(src)[k];
    }
}
}  // namespace trc

extern "C" __global__ void __launch_bounds__(trc::FILS_BRUT)
copier_brut(const uint8_t* __restrict__ partie, uint8_t* __restrict__ emplacement, trc_dims_expert dims,
            uint32_t* __restrict__ controle) {
    using namespace trc;
    const uint32_t j = blockIdx.y;
    const uint32_t R = choisir(dims.lignes, j), C = choisir(dims.colonnes, j);
    const uint32_t B = C / 32u, nblocs = R * B;
    constexpr uint8_t sortes[4] = {SORTE_CODES_BRUTS, SORTE_ECHELLES_BRUTES, SORTE_BIAIS, 0};
    DescFlux f[4];
    const bool bon = C % 32u == 0 && B > 0 && R > 0 && trouver_flux_n(partie, sortes, 3, j, f) &&
                     f[0].produits == 16u * nblocs && f[0].longueur >= 16u * nblocs && f[1].produits == nblocs &&
                     f[1].longueur >= nblocs && f[2].produits == 4u * R && f[2].longueur >= 4u * R;
    if (!bon) {
        if (threadIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    const trc_disposition disp = disposition(dims, j);
    uint8_t* mat = emplacement + disp.base;
    const uint32_t n_codes = nblocs, n_ech = (nblocs + 15u) / 16u, n_biais = (4u * R + 15u) / 16u;
    const uint32_t total = n_codes + n_ech + n_biais;
    for (uint32_t u = blockIdx.x * blockDim.x + threadIdx.x; u < total; u += gridDim.x * blockDim.x) {
        if (u < n_codes)
            copier_unite(f[0].p, mat, u, 16u * nblocs);
        else if (u < n_codes + n_ech)
            copier_unite(f[1].p, mat + disp.echelles, u - n_codes, nblocs);
        else
            copier_unite(f[2].p, mat + disp.biais, u - n_codes - n_ech, 4u * R);
    }
}

// ============================================================================ GEMVs, reference order
//
// Operation-order contract (the bits of the reference's gemv_mxfp4 / gemv_f32, gemv.cuh:61-126,
// passe.cuh:104-130), for row r of y = W x + b:
//   MXFP4: P(b) = fma chain from 0 over bytes i = 0..15 of block b's 16 code bytes, each byte's low
//          nibble times x[32b + i] then its high nibble times x[32b + 16 + i], with the doubled E2M1
//          values (exact: 2 * {0, .5, 1, 1.5, 2, 3, 4, 6}, code 8 = -0);
//          A(l) = fma chain from 0 over blocks b = l, l + 32, l + 64, ... < B of 2^(e_b - 128) * P(b);
//   f32:   A(l) = fma chain from 0 over quads c = l, l + 32, ... < C/4 of w[4c + k] * x[4c + k], k = 0..3;
//   y[r] = S + b[r] (f32 add; no bias term when b is absent), S the pairwise tree over l = 0..31:
//          pairs at lane distance 16, then 8, 4, 2, 1 (every lane of the tree ends with the same S).
// Mapping here: a 32-lane half-wavefront owns a row (l = its lane), two rows per half for MXFP4
// (the x loads of a block serve both); E2M1 pairs are expanded by v_cvt_scalef32_pk_f32_fp4 (scale
// 2: the doubled values); the tree runs on ds_swizzle (xor masks within 32 lanes); the loads of a
// lane's next block are issued before the current block's arithmetic.
namespace trc {

constexpr uint32_t GEMV_LIGNES_PAR_DEMI = 2;

// S: the xor tree over a half-wavefront's 32 lanes.
__device__ __forceinline__ float arbre_32(float v) {
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));  // xor 16
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x201F));  // xor 8
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x101F));  // xor 4
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x081F));  // xor 2
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x041F));  // xor 1
    return v;
}

// Bytes 4t .. 4t + 3 of a block (code word t) continuing the chain s: byte 4t + k pairs with
// x[4t + k] (low nibble) and x[16 + 4t + k] (high nibble), i.e. xa[k] and xb[k].
__device__ __forceinline__ float chaine_mot(uint32_t mot, const f32x4 xa, const f32x4 xb, float s) {
    const f32x2 w0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(mot, 2.0f, 0);
    const f32x2 w1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(mot, 2.0f, 1);
    const f32x2 w2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(mot, 2.0f, 2);
    const f32x2 w3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(mot, 2.0f, 3);
    s = fmaf(w0.x, xa.x, s);
    s = fmaf(w0.y, xb.x, s);
    s = fmaf(w1.x, xa.y, s);
    s = fmaf(w1.y, xb.y, s);
    s = fmaf(w2.x, xa.z, s);
    s = fmaf(w2.y, xb.z, s);
    s = fmaf(w3.x, xa.w, s);
    s = fmaf(w3.y, xb.w, s);
    return s;
}

// P(b) for one block: q its 16 code bytes, xs its 32 x values as 8 float4.
__device__ __forceinline__ float chaine_bloc(const u32x4 q, const f32x4 (&xs)[8]) {
    float s = chaine_mot(q.x, xs[0], xs[4], 0.0f);
    s = chaine_mot(q.y, xs[1], xs[5], s);
    s = chaine_mot(q.z, xs[2], xs[6], s);
    return chaine_mot(q.w, xs[3], xs[7], s);
}

struct BlocGemv {
    u32x4 q[GEMV_LIGNES_PAR_DEMI];
    uint32_t e[GEMV_LIGNES_PAR_DEMI];
    f32x4 xs[8];
};

// Rows r0, r0 + 1 of an MXFP4 matrix in its slot (rows past R are read as row R - 1 and not written).
__device__ __forceinline__ void gemv_mxfp4_demi(const uint8_t* __restrict__ mat, const float* __restrict__ x,
                                                float* __restrict__ y, uint32_t R, uint32_t C, uint32_t r0,
                                                uint32_t l) {
    const uint32_t B = C / 32u;
    const trc_disposition d = disposition_matrice(R, C);
    const gptr<u32x4> codes = glob<u32x4>(mat);
    const gptr<uint8_t> ech = glob<uint8_t>(mat + d.echelles);
    const gptr<f32x4> x4 = glob<f32x4>(x);
    uint64_t base[GEMV_LIGNES_PAR_DEMI];
#pragma unroll
    for (uint32_t i = 0; i < GEMV_LIGNES_PAR_DEMI; ++i) base[i] = uint64_t(min(r0 + i, R - 1u)) * B;
    auto charger = [&](uint32_t b, BlocGemv& c) {
#pragma unroll
        for (uint32_t i = 0; i < GEMV_LIGNES_PAR_DEMI; ++i) {
            c.q[i] = codes[base[i] + b];
            c.e[i] = ech[base[i] + b];
        }
#pragma unroll
        for (uint32_t k = 0; k < 8; ++k) c.xs[k] = x4[8u * b + k];
    };
    float acc[GEMV_LIGNES_PAR_DEMI] = {};
    BlocGemv cur;
    if (l < B) charger(l, cur);
    for (uint32_t b = l; b < B; b += 32u) {
        BlocGemv suiv;
        charger(min(b + 32u, B - 1u), suiv);  // unconditional (the last one reloads a block): no wait of
                                              // the current block's arithmetic covers these loads
#pragma unroll
        for (uint32_t i = 0; i < GEMV_LIGNES_PAR_DEMI; ++i)
            acc[i] = fmaf(echelle_e8m0(cur.e[i]), chaine_bloc(cur.q[i], cur.xs), acc[i]);
        cur = suiv;
    }
    const gptr<float> biais = glob<float>(mat + d.biais);
#pragma unroll
    for (uint32_t i = 0; i < GEMV_LIGNES_PAR_DEMI; ++i) {
        const float s = arbre_32(acc[i]);
        if (l == 0u && r0 + i < R) y[r0 + i] = s + biais[r0 + i];
    }
}

// The same rows for matrices of at most GEMV_X_COLONNES columns, x staged in LDS once per block of
// FILS threads (FILS / 32 halves of PD rows each), every code and scale load of a lane issued
// before the block's barrier. A lane's blocks are l, l + 32, l + 64 (B <= 96); the arithmetic of
// each row is gemv_mxfp4_demi's, so the bits are the same whatever the block shape. x lies in LDS
// as 144 bytes per block (32 f32 and 16 bytes of padding): lane l's reads of its block start 4
// banks past lane l - 1's, so each group of 8 lanes covers the 32 banks once. The scales of a
// half's rows, contiguous in the slot, come in as 4-byte words (the vector memory unit takes as
// long over a byte load as over a 16-byte one) and are read back from LDS byte by byte.
constexpr uint32_t GEMV_X_BLOCS = 3;                            // blocks per lane at most
constexpr uint32_t GEMV_X_COLONNES = 32u * 32u * GEMV_X_BLOCS;  // 3072
constexpr uint32_t GEMV_X_PAS = 144;                            // LDS bytes per block of x

template <uint32_t FILS, uint32_t PD>  // threads per block, rows per half-wavefront
struct FormeGemvX {
    static constexpr uint32_t DEMIS = FILS / 32u;
    static constexpr uint32_t LIGNES = DEMIS * PD;                              // rows per block
    static constexpr uint32_t MOTS_ECH = PD * 32u * GEMV_X_BLOCS / 4u + 1u;     // scale words per half
    static constexpr uint32_t ECH_DEMI = 4u * MOTS_ECH;
    static constexpr uint32_t NE = (MOTS_ECH + 31u) / 32u;                     // scale words per lane
    static constexpr uint32_t NX = (GEMV_X_COLONNES / 4u + FILS - 1u) / FILS;  // float4 of x per thread
    static constexpr uint32_t LDS = (GEMV_X_COLONNES / 32u) * GEMV_X_PAS + DEMIS * ECH_DEMI;
};

template <uint32_t FILS, uint32_t PD, uint32_t NB>  // NB: blocks per lane, ceil(B / 32)
__device__ __forceinline__ void gemv_mxfp4_x_lds_n(const uint8_t* __restrict__ mat, const float* __restrict__ x,
                                                   float* __restrict__ y, uint32_t R, uint32_t C, uint32_t r_bloc,
                                                   uint8_t* __restrict__ xl) {
    using F = FormeGemvX<FILS, PD>;
    const uint32_t B = C / 32u;
    const uint32_t l = threadIdx.x & 31u;
    const uint32_t r0 = r_bloc + (threadIdx.x >> 5) * PD;
    const trc_disposition d = disposition_matrice(R, C);
    const gptr<u32x4> codes = glob<u32x4>(mat);
    const gptr<uint32_t> ech32 = glob<uint32_t>(mat + d.echelles);  // 256-aligned region of R * B bytes
    const gptr<f32x4> x4 = glob<f32x4>(x);
    // x first, then the scale words: the waits before their LDS stores leave the code loads, issued
    // after them, in flight
    f32x4 xv[F::NX];
#pragma unroll
    for (uint32_t k = 0; k < F::NX; ++k) xv[k] = x4[min(threadIdx.x + k * FILS, C / 4u - 1u)];
    // the half's scale bytes [r0 B, (r0 + PD) B) as the words from the one holding byte r0 B
    const uint32_t o0 = r0 * B, a0 = o0 >> 2, dernier_mot = (R * B + 3u) / 4u - 1u;
    uint32_t ev[F::NE];
#pragma unroll
    for (uint32_t k = 0; k < F::NE; ++k) ev[k] = ech32[min(a0 + l + 32u * k, dernier_mot)];
    u32x4 q[PD][NB];
    // block by block, so that the arithmetic of a lane's first block waits for its loads only
    // (vector memory completes in order)
#pragma unroll
    for (uint32_t j = 0; j < NB; ++j) {
        const uint32_t b = min(l + 32u * j, B - 1u);  // past B: a block reloaded, never used
#pragma unroll
        for (uint32_t i = 0; i < PD; ++i) q[i][j] = codes[uint64_t(min(r0 + i, R - 1u)) * B + b];
    }
#pragma unroll
    for (uint32_t k = 0; k < F::NX; ++k) {
        const uint32_t g = threadIdx.x + k * FILS;  // float4 g: block g / 8, quarter g % 8
        if (g < C / 4u) *reinterpret_cast<f32x4*>(xl + (g >> 3) * GEMV_X_PAS + 16u * (g & 7u)) = xv[k];
    }
    uint8_t* el = xl + (GEMV_X_COLONNES / 32u) * GEMV_X_PAS + (threadIdx.x >> 5) * F::ECH_DEMI;
#pragma unroll
    for (uint32_t k = 0; k < F::NE; ++k)
        if (4u * (l + 32u * k) < F::ECH_DEMI) *reinterpret_cast<uint32_t*>(el + 4u * (l + 32u * k)) = ev[k];
    __syncthreads();
    // scale of row i, block b: byte (o0 & 3) + i B + b of the half's words (rows past R: unused)
    const uint8_t* el_r = el + (o0 & 3u);
    float acc[PD] = {};
#pragma unroll
    for (uint32_t j = 0; j < NB; ++j) {
        const uint32_t b = l + 32u * j;
        if (b < B) {
            // word by word (x values 4t .. 4t + 3 and 16 + 4t ..): each row's chain keeps
            // chaine_bloc's order, and only two float4 of x are live at a time
            float p[PD] = {};
#pragma unroll
            for (uint32_t t = 0; t < 4; ++t) {
                const f32x4 xa = *reinterpret_cast<const f32x4*>(xl + b * GEMV_X_PAS + 16u * t);
                const f32x4 xb = *reinterpret_cast<const f32x4*>(xl + b * GEMV_X_PAS + 64u + 16u * t);
#pragma unroll
                for (uint32_t i = 0; i < PD; ++i) p[i] = chaine_mot(q[i][j][t], xa, xb, p[i]);
            }
#pragma unroll
            for (uint32_t i = 0; i < PD; ++i) acc[i] = fmaf(echelle_e8m0(el_r[i * B + b]), p[i], acc[i]);
        }
    }
    const gptr<float> biais = glob<float>(mat + d.biais);
#pragma unroll
    for (uint32_t i = 0; i < PD; ++i) {
        const float s = arbre_32(acc[i]);
        if (l == 0u && r0 + i < R) y[r0 + i] = s + biais[r0 + i];
    }
}

// gemv_mxfp4_x_lds_n for the matrix's blocks per lane (uniform over the block), so that only the
// loads a lane can use are held in registers.
template <uint32_t FILS, uint32_t PD>
__device__ __forceinline__ void gemv_mxfp4_x_lds(const uint8_t* __restrict__ mat, const float* __restrict__ x,
                                                 float* __restrict__ y, uint32_t R, uint32_t C, uint32_t r_bloc,
                                                 uint8_t* __restrict__ xl) {
    const uint32_t nb = (C / 32u + 31u) / 32u;
    if (nb <= 1u)
        gemv_mxfp4_x_lds_n<FILS, PD, 1>(mat, x, y, R, C, r_bloc, xl);
    else if (nb == 2u)
        gemv_mxfp4_x_lds_n<FILS, PD, 2>(mat, x, y, R, C, r_bloc, xl);
    else
        gemv_mxfp4_x_lds_n<FILS, PD, 3>(mat, x, y, R, C, r_bloc, xl);
}

}  // namespace trc

// y = W x + b, x in LDS (C <= GEMV_X_COLONNES): FormeGemvX<FILS, PD>::LIGNES rows per block.
template <uint32_t FILS, uint32_t PD>
__global__ void __launch_bounds__(FILS)
gemv_mxfp4_x(const uint8_t* __restrict__ matrice, const float* __restrict__ x, float* __restrict__ y, uint32_t R,
             uint32_t C) {
    __shared__ __attribute__((aligned(16))) uint8_t xl[trc::FormeGemvX<FILS, PD>::LDS];
    trc::gemv_mxfp4_x_lds<FILS, PD>(matrice, x, y, R, C, blockIdx.x * trc::FormeGemvX<FILS, PD>::LIGNES, xl);
}

// The batch form: grid y = product; a product wider than GEMV_X_COLONNES takes gemv_mxfp4_demi for
// the same rows (each half-wavefront two at a time). Both branches are uniform over the block (its
// rows belong to one product), so the barrier of the LDS form is reached by all.
template <uint32_t FILS, uint32_t PD>
__global__ void __launch_bounds__(FILS) gemv_mxfp4_lot_x(const trc::DescGemv* __restrict__ descs) {
    using F = trc::FormeGemvX<FILS, PD>;
    __shared__ __attribute__((aligned(16))) uint8_t xl[F::LDS];
    const trc::DescGemv dsc = descs[blockIdx.y];
    const uint32_t r_bloc = blockIdx.x * F::LIGNES;
    if (r_bloc >= dsc.lignes || dsc.colonnes % 32u != 0) return;
    if (dsc.colonnes > trc::GEMV_X_COLONNES) {
        for (uint32_t r0 = r_bloc + (threadIdx.x >> 5) * trc::GEMV_LIGNES_PAR_DEMI;
             r0 < min(r_bloc + F::LIGNES, dsc.lignes); r0 += F::DEMIS * trc::GEMV_LIGNES_PAR_DEMI)
            trc::gemv_mxfp4_demi(reinterpret_cast<const uint8_t*>(dsc.matrice), reinterpret_cast<const float*>(dsc.x),
                                 reinterpret_cast<float*>(dsc.y), dsc.lignes, dsc.colonnes, r0, threadIdx.x & 31u);
        return;
    }
    trc::gemv_mxfp4_x_lds<FILS, PD>(reinterpret_cast<const uint8_t*>(dsc.matrice), reinterpret_cast<const float*>(dsc.x),
                                    reinterpret_cast<float*>(dsc.y), dsc.lignes, dsc.colonnes, r_bloc, xl);
}

// y = W x + b for one slot matrix: 8 halves x 2 rows per block of 256 threads.
extern "C" __global__ void __launch_bounds__(trc::GEMV_FILS)
gemv_mxfp4(const uint8_t* __restrict__ matrice, const float* __restrict__ x, float* __restrict__ y, uint32_t R,
           uint32_t C) {
    const uint32_t r0 = (blockIdx.x * (trc::GEMV_FILS / 32u) + (threadIdx.x >> 5)) * trc::GEMV_LIGNES_PAR_DEMI;
    if (r0 >= R || C % 32u != 0) return;
    trc::gemv_mxfp4_demi(matrice, x, y, R, C, r0, threadIdx.x & 31u);
}

// Independent products (e.g. the 12 matrices of a layer's 4 experts) in one launch: grid y = product.
extern "C" __global__ void __launch_bounds__(trc::GEMV_FILS) gemv_mxfp4_lot(const trc::DescGemv* __restrict__ descs) {
    const trc::DescGemv dsc = descs[blockIdx.y];
    const uint32_t r0 = (blockIdx.x * (trc::GEMV_FILS / 32u) + (threadIdx.x >> 5)) * trc::GEMV_LIGNES_PAR_DEMI;
    if (r0 >= dsc.lignes || dsc.colonnes % 32u != 0) return;
    trc::gemv_mxfp4_demi(reinterpret_cast<const uint8_t*>(dsc.matrice), reinterpret_cast<const float*>(dsc.x),
                         reinterpret_cast<float*>(dsc.y), dsc.lignes, dsc.colonnes, r0, threadIdx.x & 31u);
}

// y = W x (+ b), W f32 row-major: one row per half-wavefront, four quads per lane in flight.
extern "C" __global__ void __launch_bounds__(trc::GEMV_FILS)
gemv_f32(const float* __restrict__ W, const float* __restrict__ x, const float* __restrict__ biais,
         float* __restrict__ y, uint32_t R, uint32_t C) {
    using namespace trc;
    const uint32_t r = blockIdx.x * (GEMV_FILS / 32u) + (threadIdx.x >> 5);
    const uint32_t l = threadIdx.x & 31u;
    if (r >= R || C % 4u != 0) return;
    const uint32_t C4 = C / 4u;
    const gptr<f32x4> w4 = glob<f32x4>(W + uint64_t(r) * C);
    const gptr<f32x4> x4 = glob<f32x4>(x);
    constexpr uint32_t LOT = 4;
    float acc = 0.0f;
    uint32_t c = l;
    for (; c + 32u * (LOT - 1u) < C4; c += 32u * LOT) {  // whole batches: every load goes out first
        f32x4 w[LOT], xv[LOT];
#pragma unroll
        for (uint32_t u = 0; u < LOT; ++u) {
            w[u] = w4[c + 32u * u];
            xv[u] = x4[c + 32u * u];
        }
#pragma unroll
        for (uint32_t u = 0; u < LOT; ++u) {
            acc = fmaf(w[u].x, xv[u].x, acc);
            acc = fmaf(w[u].y, xv[u].y, acc);
            acc = fmaf(w[u].z, xv[u].z, acc);
            acc = fmaf(w[u].w, xv[u].w, acc);
        }
    }
    for (; c < C4; c += 32u) {
        const f32x4 w = w4[c], xv = x4[c];
        acc = fmaf(w.x, xv.x, acc);
        acc = fmaf(w.y, xv.y, acc);
        acc = fmaf(w.z, xv.z, acc);
        acc = fmaf(w.w, xv.w, acc);
    }
    const float s = arbre_32(acc);
    if (l == 0u) y[r] = biais != nullptr ? s + biais[r] : s;
}

// =========================================================================== router, SwiGLU, combine

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
    hipLaunchKernelGGL(decoder_codes, dim3(g2[0], 3, 1), dim3(trc::FILS_CODES_SLOT), 0, f, p, e, l, *dims, c);
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
    hipLaunchKernelGGL(decoder_codes_lot, dim3(g2[0], 3, n), dim3(trc::FILS_CODES_SLOT), 0, f, d, *dims);
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

namespace {

template <uint32_t FILS, uint32_t PD>
int lancer_gemv_lot_x_forme(const trc::DescGemv* descs, uint32_t n, uint32_t lignes_max, hipStream_t f) {
    constexpr uint32_t L = trc::FormeGemvX<FILS, PD>::LIGNES;
    hipLaunchKernelGGL((gemv_mxfp4_lot_x<FILS, PD>), dim3((lignes_max + L - 1) / L, n), dim3(FILS), 0, f, descs);
    return trc::apres_lancement("gemv_mxfp4_lot_x");
}

// The block shape of a batch of n products of at most lignes_max rows: one row per
// half-wavefront (32 VGPRs, so that a CU holds many wavefronts whose loads and arithmetic overlap),
// 16 halves per block, or 8 when that leaves fewer than 512 blocks. Measured on MI355X over 4, 8
// and 12 gpt-oss matrices against 2 and 4 rows per half and 4 to 32 halves per block.
int lancer_gemv_lot_x(const trc::DescGemv* descs, uint32_t n, uint32_t lignes_max, hipStream_t f) {
    if (uint64_t(n) * ((lignes_max + 15u) / 16u) < 512u) return lancer_gemv_lot_x_forme<256, 1>(descs, n, lignes_max, f);
    return lancer_gemv_lot_x_forme<512, 1>(descs, n, lignes_max, f);
}

}  // namespace

extern "C" int trc_gemv(trc_vue matrice, trc_vue x, trc_vue y, uint32_t lignes, uint32_t colonnes, void* flux) {
    TRC_VERIFIER(lignes > 0 && colonnes > 0 && colonnes % 32 == 0, "forme %u x %u", lignes, colonnes);
    const uint64_t pas = trc::disposition_matrice(lignes, colonnes).pas;
    TRC_VERIFIER(matrice.adresse != 0 && matrice.octets >= pas, "matrice de %llu o, %llu o demandes",
                 (unsigned long long)matrice.octets, (unsigned long long)pas);
    TRC_VERIFIER(matrice.adresse % 256 == 0, "matrice non alignee sur 256");
    TRC_VERIFIER(x.adresse != 0 && x.octets >= 4ull * colonnes && x.adresse % 16 == 0,
                 "x trop court ou non aligne sur 16");
    TRC_VERIFIER(y.adresse != 0 && y.octets >= 4ull * lignes, "y trop court");
    if (colonnes <= trc::GEMV_X_COLONNES) {
        constexpr uint32_t L = trc::FormeGemvX<256, 1>::LIGNES;  // a single product: 8 rows per block
        hipLaunchKernelGGL((gemv_mxfp4_x<256, 1>), dim3((lignes + L - 1) / L), dim3(256), 0, flux_de(flux),
                           reinterpret_cast<const uint8_t*>(matrice.adresse), reinterpret_cast<const float*>(x.adresse),
                           reinterpret_cast<float*>(y.adresse), lignes, colonnes);
        return trc::apres_lancement("gemv_mxfp4_x");
    }
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
    return lancer_gemv_lot_x(reinterpret_cast<const trc::DescGemv*>(descs.adresse), n, lignes_max, flux_de(flux));
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
    constexpr uint32_t lignes_bloc = trc::GEMV_FILS / 32u;  // one row per half-wavefront
    hipLaunchKernelGGL(gemv_f32, dim3((lignes + lignes_bloc - 1) / lignes_bloc),
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
