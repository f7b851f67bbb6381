// prefill.hip — batched prefill of a resident MoE layer on gfx950 (T positions, top-k each): every
// chosen expert is rANS-decoded once, band of rows by band of rows, into LDS as MXFP4 (E2M1 codes,
// E8M0 block scales) and multiplied against all the positions that chose it on the bf16 MFMA
// (v_mfma_f32_16x16x32_bf16, fp32 accumulation), the weights converted to bf16 (exactly) where they
// are read and the activations split into exact bf16 pieces. The reference runs the same layer as
// one decode per chosen expert then one GEMV chain per (position, slot) (trc-ordo/src/lib.rs:782-945,
// expert_pos and combiner_pos, trc-modele/src/lib.rs:688-710). Launches, one stream:
//
//   prefill_grouper       (position, slot) pairs grouped by expert, in position order within an
//                         expert (the reference's par_expert lists, trc-ordo/src/lib.rs:815-823);
//   prefill_quant_x       each position's x split into bf16 pieces (hi + mid + lo = x);
//   fusion_echelles       (prefill mode) DELTA -> block entries of every chosen expert's matrices;
//   prefill_mfma_gu       gate and up: bands decoded into LDS, bf16 MFMA (the weights converted from
//                         MXFP4 where they are read) against the expert's positions, + bias -> gu;
//
// Streams whose CODES_CTX tiles are longer than the 16 macro-steps a band holds in registers (the
// reference encoder writes 256, rans.rs:32) take two slot-decoder launches instead of the DELTA pass
// (prefill_emplacements_echelles, prefill_emplacements_codes: every chosen expert decoded once into
// a slot of the reference's layout, all of them at once, so the long chains run side by side), and
// the band kernels copy their band's codes and scales from the slot instead of decoding them.
//   prefill_swiglu_quant  act = swiglu_oai(gate, up) per pair, split into bf16 pieces;
//   prefill_mfma_bas      down -> s, one row of D per pair (the reference's pos.s layout), bf16 MFMA;
//   prefill_combiner      x_i += ((w0 s_i0 + w1 s_i1) + ...) in slot order, no FMA.
//
// Activations in bf16 pieces. A row v of f32 activations (x for gate and up, act for down) is
// written as v = hi + mid + lo with hi = bf16(v), mid = bf16(v - hi) and lo = bf16(v - hi - mid),
// each difference exact in f32: hi leaves at most 16 significant bits, mid at most 8, which lo
// holds. A weight, e2m1 x 2^(e - 127), is exact in bf16 too, so every product of
// v_mfma_f32_16x16x32_bf16 is exact and y differs from the f32 GEMV only by the fp32 accumulation
// order. Pieces that are zero for every row of the call are skipped: bf16 activations need one.
//
// MFMA operand layout (v_mfma_f32_16x16x32_bf16): lane g*16 + r holds 8 K values of row r of A and
// the same 8 K values of column r of B; C: lane g*16 + n holds rows 4 g .. 4 g + 3 of column n. A
// weight block is 16 code bytes, byte i holding weights i (low nibble) and 16 + i, so lane g takes
// bytes 4g .. 4g + 3 and a piece block stores value (j >> 1) + 16 (j & 1) at position j.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>

#include "anneau.hpp"
#include "chrono.hpp"
#include "codes.hpp"
#include "commun.hpp"
#include "emplacement.hpp"
#include "erreurs.hpp"
#include "fusion_corps.hpp"
#include "selection.hpp"

namespace trc {

constexpr uint32_t PF_FILS = 1024;        // 16 wavefronts: 32 tiles decoded per band
constexpr uint32_t PF_FILS_CODES_SLOT = 1024;  // long tiles' CODES_CTX slot decoder: 32 tiles per block
constexpr uint32_t PF_NMAX = 16;          // macro-steps per CODES_CTX tile held in registers
constexpr uint32_t PF_PIECES_BF = 3;      // bf16 pieces per activation block
constexpr uint32_t PF_Q_FILS = 256;       // threads per block of the piece kernels (16 per 32-value block)
constexpr uint32_t PF_BP_MAX = 128;       // blocks per row at most (4096 columns)
constexpr uint32_t PF_PAIRES_MAX = 16384; // positions x k per call
constexpr uint32_t ECHELLE_UN = 127u;     // E8M0 1.0

constexpr uint32_t PF_FILS_RAPIDE = 1024;   // slot decoder with each tile's DELTA: 32 tiles per block
constexpr uint32_t PF_PAIRES_RAPIDE = 8;    // its tile pairs per wavefront (the LUT staging amortised over them)
constexpr uint32_t PF_LOT_COPIE = 8;     // 16-byte loads per thread in flight when a band is copied from a slot
constexpr uint32_t PF_LOT_ECH = PF_LOT_COPIE / 4u;  // scale words with them (4 blocks per word)
constexpr uint32_t PF_TOURS = 2;          // decode rounds per band: a band's tiles are at most 64
constexpr uint32_t PF_RB_MAX = 80;         // rows per band
constexpr uint32_t PF_RT_MAX = PF_RB_MAX / 16u;  // row tiles per band

// LDS of prefill_mfma after the decode (every region of the decode is free then): codes [RB][B][16 B]
// at 0 (rows of exactly B blocks), scales [RB][B] after them, then the partial sums of the MFMA phase,
// half the waves' at a time (RB/16 row tiles x 8 waves x 64 lanes x 16 B).
constexpr uint32_t PF_A = 0;
__host__ __device__ inline uint32_t pf_sa(uint32_t rb, uint32_t b) { return rb * b * 16u; }
__host__ __device__ inline uint32_t pf_part(uint32_t rb, uint32_t b) { return (pf_sa(rb, b) + rb * b + 15u) & ~15u; }
__host__ __device__ inline uint32_t pf_part_octets(uint32_t rb) { return (rb / 16u) * 8u * 64u * 16u; }
__host__ __device__ inline bool pf_lds_tient(uint32_t rb, uint32_t b) { return pf_part(rb, b) + pf_part_octets(rb) <= LDS_GEMV; }

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

struct ParamsPrefill {
    uint64_t repertoire;   // MatricePartie[E][3] of the mounted layer
    uint64_t ech;          // block entries of matrix (e, j) at ech + (e*3 + j) * pas_ech
    uint64_t pas_ech;
    uint64_t compte;       // u32[E] pairs per expert
    uint64_t debut;        // u32[E] first pair of expert e in `paires`
    uint64_t paires;       // u32[T*k] pair c = i*k + slot, grouped by expert
    uint64_t pieces;       // u32[4]: [0] bf16 pieces used by x, [1] by act
    uint64_t indices;      // u32[T*k] chosen experts
    uint64_t poids;        // f32[T*k] their weights
    uint64_t x;            // f32[T][C]
    uint64_t residus;      // f32[T][D]
    uint64_t xb;           // x pieces, bf16: xb[((i*PF_PIECES_BF + p)*bx + b)*32 + j], j in the order
                           // of the weight block's nibbles: x[32 b + (j >> 1) + 16 (j & 1)]; block
                           // b = C/32 (the last of the bx = C/32 + 1) is zero
    uint64_t gu;           // f32[T*k][2][R]
    uint64_t ab;           // act pieces per pair, like xb with bact blocks per piece row
    uint64_t s;            // f32[T*k][D]
    uint32_t lignes[3], colonnes[3];
    uint32_t rb[3];        // rows per band (16, 32, 64 or 80)
    uint32_t T, k, E, D;
    uint32_t bx, bact;     // blocks per piece row of x and act: C/32 + 1, R/32 + 1
    uint32_t quatre;       // the combine takes 4 rows per thread (D % 4 == 0, residus 16-byte aligned)
    uint64_t emplacements; // long tiles: expert e's slot (reference layout) at emplacements + e * pas_emplacement,
                           // decoded by the slot decoders; 0: the band kernels decode their tiles
    uint64_t pas_emplacement;
};

// The slot layout of a prefill's experts (the reference's, abi.rs:76-122).
__device__ __forceinline__ trc_dims_expert dims_prefill(const ParamsPrefill& pp) {
    trc_dims_expert d;
#pragma unroll
    for (uint32_t j = 0; j < 3; ++j) {
        d.lignes[j] = pp.lignes[j];
        d.colonnes[j] = pp.colonnes[j];
    }
    return d;
}

// Splits values q and q + 16 of a 32-value block into PF_PIECES_BF bf16 pieces: word q of each
// 64-byte piece block (piece stride `pas` bytes) holds value q (low half) and q + 16 (high half).
// Returns the pieces that are not both zero. An infinite or NaN value stays whole in hi (its
// residual is set to 0), so a product with it is what the f32 product is.
__device__ __forceinline__ uint32_t pieces_bf16(float a0, float a1, uint8_t* dst, uint64_t pas) {
    uint32_t P = 0;
#pragma unroll
    for (uint32_t p = 0; p < PF_PIECES_BF; ++p) {
        const __bf16 h0 = __bf16(a0), h1 = __bf16(a1);
        const uint32_t b0 = __builtin_bit_cast(uint16_t, h0), b1 = __builtin_bit_cast(uint16_t, h1);
        const float f0 = __uint_as_float(b0 << 16), f1 = __uint_as_float(b1 << 16);
        a0 = __builtin_isfinite(f0) ? a0 - f0 : 0.0f;  // exact
        a1 = __builtin_isfinite(f1) ? a1 - f1 : 0.0f;
        const uint32_t mot = b0 | (b1 << 16);
        *reinterpret_cast<uint32_t*>(dst + p * pas) = mot;
        if (mot & 0x7FFF7FFFu) P = p + 1u;
    }
    return P;
}

__device__ __forceinline__ uint32_t max_vague(uint32_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = max(v, uint32_t(__shfl_xor(int(v), d)));
    return v;
}

// *compteur = max(*compteur, the wave's P). The counter only grows, so a wave whose P does not
// exceed the value it reads needs no atomic: most waves of a call then leave the address alone.
__device__ __forceinline__ void noter_pieces(uint32_t* compteur, uint32_t P) {
    P = max_vague(P);
    if (__lane_id() == 0 && P && P > __hip_atomic_load(compteur, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
        atomicMax(compteur, P);
}

}  // namespace trc

using trc::ParamsPrefill;

// One block of 1024 threads groups the pairs by expert, in position order within an expert. Wave w
// takes the pairs of its contiguous share, 64 at a time: the lanes holding the same expert find
// each other with one ballot per bit of the index, and a pair's rank among the wave's earlier pairs
// of its expert is the count of those lanes below it plus the wave's running count (kept in LDS).
// The experts' starts are an exclusive prefix of the totals; a wave's pairs of expert e follow the
// earlier waves' ones. Also clears the piece counters of the call. Indices >= E are format errors
// (the reference bails, trc-ordo/src/lib.rs:817-819) and join no list.
extern "C" __global__ void __launch_bounds__(1024)
prefill_grouper(ParamsPrefill pp, uint32_t* __restrict__ controle) {
    using namespace trc;
    constexpr uint32_t VAGUES = 16;
    __shared__ uint32_t cpt[VAGUES][EXPERTS_MAX];  // per wave: its pairs of each expert so far, then its base
    __shared__ uint16_t rang[PF_PAIRES_MAX];       // a pair's rank among its wave's pairs of its expert
    __shared__ uint32_t deb[EXPERTS_MAX];
    const uint32_t n = pp.T * pp.k, E = pp.E;
    const uint32_t* indices = reinterpret_cast<const uint32_t*>(pp.indices);
    const uint32_t lane = __lane_id(), w = threadIdx.x >> 6;
    for (uint32_t i = threadIdx.x; i < VAGUES * EXPERTS_MAX; i += blockDim.x) (&cpt[0][0])[i] = 0u;
    if (threadIdx.x < 4u) reinterpret_cast<uint32_t*>(pp.pieces)[threadIdx.x] = 0u;
    __syncthreads();
    const uint32_t par_vague = (n + VAGUES - 1u) / VAGUES;
    const uint32_t p0 = min(n, w * par_vague), p1 = min(n, p0 + par_vague);
    const uint64_t dessous = (uint64_t(1) << lane) - 1u;
    uint32_t mauvais = 0;
    for (uint32_t b = p0; b < p1; b += 64u) {  // wave-uniform
        const uint32_t p = b + lane;
        const uint32_t e = p < p1 ? indices[p] : 0xFFFFFFFFu;
        const bool valide = e < E;
        mauvais += (p < p1 && !valide) ? 1u : 0u;
        uint64_t meme = __builtin_amdgcn_ballot_w64(valide);
#pragma unroll
        for (uint32_t bit = 0; bit < 8; ++bit) {  // E <= 256
            const bool un = (e >> bit) & 1u;
            const uint64_t v = __builtin_amdgcn_ballot_w64(un);
            meme &= un ? v : ~v;
        }
        const uint32_t avant = __popcll(meme & dessous);
        const uint32_t ee = valide ? e : 0u;
        const uint32_t deja = valide ? cpt[w][ee] : 0u;
        if (valide) rang[p] = uint16_t(deja + avant);
        // the group's highest lane raises the wave's count of the expert
        if (valide && (meme >> lane) == 1u) cpt[w][ee] = deja + avant + 1u;
    }
    mauvais = somme_vague_u32(mauvais);
    if (lane == 0 && mauvais) atomicAdd(&controle[CTL_FORMAT], mauvais);
    __syncthreads();
    // per expert e (thread e): total and the waves' bases, then the experts' exclusive prefix
    uint32_t total = 0;
    if (threadIdx.x < EXPERTS_MAX) {
        for (uint32_t v = 0; v < VAGUES; ++v) {
            const uint32_t c = cpt[v][threadIdx.x];
            cpt[v][threadIdx.x] = total;
            total += c;
        }
        deb[threadIdx.x] = total;
    }
    __syncthreads();
    if (threadIdx.x < 64u) {  // exclusive prefix over experts, 4 per lane
        uint32_t t[EXPERTS_MAX / 64];
        uint32_t local = 0;
#pragma unroll
        for (uint32_t q = 0; q < EXPERTS_MAX / 64; ++q) {
            t[q] = deb[threadIdx.x * (EXPERTS_MAX / 64) + q];
            local += t[q];
        }
        uint32_t incl = local;
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t u = uint32_t(__shfl_up(int(incl), d));
            if (int(threadIdx.x) >= d) incl += u;
        }
        uint32_t s0 = incl - local;
#pragma unroll
        for (uint32_t q = 0; q < EXPERTS_MAX / 64; ++q) {
            const uint32_t ee = threadIdx.x * (EXPERTS_MAX / 64) + q;
            deb[ee] = s0;
            if (ee < E) {
                reinterpret_cast<uint32_t*>(pp.debut)[ee] = s0;
                reinterpret_cast<uint32_t*>(pp.compte)[ee] = t[q];
            }
            s0 += t[q];
        }
    }
    __syncthreads();
    uint32_t* paires = reinterpret_cast<uint32_t*>(pp.paires);
    for (uint32_t b = p0; b < p1; b += 64u) {
        const uint32_t p = b + lane;
        if (p < p1) {
            const uint32_t e = indices[p];
            if (e < E) paires[deb[e] + cpt[w][e] + rang[p]] = p;
        }
    }
}

// x pieces: block i (position i); thread g takes, for (b, q) = (g / 16, g % 16), g + 256 k, values q
// and q + 16 of block b (block B gets zeros), so that a wave's loads and stores are contiguous.
extern "C" __global__ void __launch_bounds__(trc::PF_Q_FILS)
prefill_quant_x(ParamsPrefill pp) {
    using namespace trc;
    const uint32_t i = blockIdx.x;
    const uint32_t C = pp.colonnes[0], B = C / 32u, Bx = pp.bx;
    uint32_t P = 0;
    for (uint32_t g = threadIdx.x; g < Bx * 16u; g += PF_Q_FILS) {
        const uint32_t b = g >> 4, q = g & 15u;
        const float* x = reinterpret_cast<const float*>(pp.x) + uint64_t(i) * C + 32u * b + q;
        const float a0 = b < B ? x[0] : 0.0f, a1 = b < B ? x[16] : 0.0f;
        P = max(P, pieces_bf16(a0, a1,
                               reinterpret_cast<uint8_t*>(pp.xb) + (uint64_t(i) * PF_PIECES_BF * Bx + b) * 64u + 4u * q,
                               uint64_t(Bx) * 64u));
    }
    noter_pieces(reinterpret_cast<uint32_t*>(pp.pieces), P);
}

// act pieces: block c (pair c); thread g takes, for (b, q) = (g / 16, g % 16), g + 256 k, rows
// 32b + q and 32b + q + 16 of act = swiglu_oai(gate, up) (block R/32 gets zeros).
extern "C" __global__ void __launch_bounds__(trc::PF_Q_FILS)
prefill_swiglu_quant(ParamsPrefill pp) {
    using namespace trc;
    const uint32_t c = blockIdx.x;
    const uint32_t R = pp.lignes[0], B2 = R / 32u, Ba = pp.bact;
    if (reinterpret_cast<const uint32_t*>(pp.indices)[c] >= pp.E) return;
    uint32_t P = 0;
    for (uint32_t g = threadIdx.x; g < Ba * 16u; g += PF_Q_FILS) {
        const uint32_t b = g >> 4, q = g & 15u;
        const float* gt = reinterpret_cast<const float*>(pp.gu) + uint64_t(c) * 2u * R + 32u * b + q;
        const float* up = gt + R;
        const float a0 = b < B2 ? swiglu_oai_f(gt[0], up[0]) : 0.0f;
        const float a1 = b < B2 ? swiglu_oai_f(gt[16], up[16]) : 0.0f;
        P = max(P, pieces_bf16(a0, a1,
                               reinterpret_cast<uint8_t*>(pp.ab) + (uint64_t(c) * PF_PIECES_BF * Ba + b) * 64u + 4u * q,
                               uint64_t(Ba) * 64u));
    }
    noter_pieces(reinterpret_cast<uint32_t*>(pp.pieces) + 1, P);
}

// Long tiles: DELTA of matrix j = blockIdx.y of expert e = blockIdx.z -> the scales and biases of
// the expert's slot, for every expert that a position chose; streams from the mounted directory,
// whose record carries the reader's checks (a failed record is a format error, counted once here
// and once by the band kernels, as the DELTA pass and the band kernels count it for short tiles).
extern "C" __global__ void __launch_bounds__(trc::FILS_ECHELLES)
prefill_emplacements_echelles(ParamsPrefill pp, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    using namespace trc;
    __shared__ LdsEchelles<FILS_ECHELLES> s;
    const uint32_t e = blockIdx.z, j = blockIdx.y;
    if (reinterpret_cast<const uint32_t*>(pp.compte)[e] == 0u) return;
    const MatricePartie m = lire_matrice_constante(pp.repertoire + uint64_t(e * 3u + j) * sizeof(MatricePartie));
    const uint32_t R = choisir(pp.lignes, j), B = choisir(pp.colonnes, j) / 32u;
    if (m.bon == 0u) {
        if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    const trc_disposition disp = disposition(dims_prefill(pp), j);
    uint8_t* mat = reinterpret_cast<uint8_t*>(pp.emplacements + uint64_t(e) * pp.pas_emplacement + disp.base);
    echelles_vers_emplacement<FILS_ECHELLES>(m.delta, m.med, m.biais, entete_de(m.delta, m.dP, m.dN, m.dT, m.dW), R, B,
                                             mat, disp, luts + uint64_t(j) * 4u * M, controle, s);
}

// Long tiles: CODES_CTX of matrix j = blockIdx.y of expert e = blockIdx.z -> the code bytes of the
// expert's slot (contexts from the slot's scales, decoded by the launch before). 1024-thread blocks:
// 32 tiles per block, the three decode tables staged once for them.
extern "C" __global__ void __launch_bounds__(trc::PF_FILS_CODES_SLOT)
prefill_emplacements_codes(ParamsPrefill pp, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    using namespace trc;
    __shared__ LdsCodesT<PF_FILS_CODES_SLOT> s;
    const uint32_t e = blockIdx.z, j = blockIdx.y;
    if (reinterpret_cast<const uint32_t*>(pp.compte)[e] == 0u) return;
    const MatricePartie m = lire_matrice_constante(pp.repertoire + uint64_t(e * 3u + j) * sizeof(MatricePartie));
    if (m.bon == 0u) return;  // counted by the DELTA launch
    const uint32_t R = choisir(pp.lignes, j), B = choisir(pp.colonnes, j) / 32u;
    const trc_disposition disp = disposition(dims_prefill(pp), j);
    uint8_t* mat = reinterpret_cast<uint8_t*>(pp.emplacements + uint64_t(e) * pp.pas_emplacement + disp.base);
    codes_vers_emplacement<PF_FILS_CODES_SLOT>(m.codes, m.med, entete_de(m.codes, m.cP, m.cN, m.cT, m.cW), R, B, mat,
                                               disp, luts + (uint64_t(j) * 4u + 1u) * M, controle, s);
}

// Tiles whose DELTA the CODES pass decodes itself (N_codes = 16 with N_delta 1 or 2, 32 with 2):
// matrix j = blockIdx.y of every chosen expert e = blockIdx.z decoded into its slot, scales and
// codes in one pass, by the CODES pass's tile machinery (read one tile ahead, each tile's DELTA
// decoded by its half-wavefront, entries in LDS; codes.hpp). The prologue issues the loads that do
// not depend on the record first (the DELTA LUT, staged in LDS for the first tiles, and the decode
// LUTs), then the record, then the first tiles' streams.
extern "C" __global__ void __launch_bounds__(trc::PF_FILS_RAPIDE)
prefill_emplacements_delta_interne(ParamsPrefill pp, const uint32_t* __restrict__ luts,
                                   uint32_t* __restrict__ controle) {
    using namespace trc;
    __shared__ __attribute__((aligned(16384))) uint8_t lds[LDS_GEMV];
    constexpr uint32_t FILS = PF_FILS_RAPIDE;
    const uint32_t e = blockIdx.z, j = blockIdx.y;
    if (uniforme32(glob<uint32_t>(reinterpret_cast<const void*>(pp.compte))[e]) == 0u) return;
    const Grille g{FILS, uniforme32(gridDim.x)};
    const uint32_t R = choisir(pp.lignes, j), C = choisir(pp.colonnes, j);
    constexpr uint32_t LOT_D = (M / 4u + FILS - 1u) / FILS;  // 16-byte groups of the DELTA LUT per thread
    u32x4 lutd_v[LOT_D];
#pragma unroll
    for (uint32_t k = 0; k < LOT_D; ++k)
        lutd_v[k] = glob<u32x4>(luts + uint64_t(j) * 4u * M)[min(k * FILS + threadIdx.x, M / 4u - 1u)];
    ChargeLutBloc<FILS> charge_lut;
    charge_lut.demarrer(luts + (uint64_t(j) * 4u + 1u) * M);
    const MatricePartie m = lire_matrice_constante(pp.repertoire + uint64_t(e * 3u + j) * sizeof(MatricePartie));
    Tache tc{};
    tc.lignes = R;
    tc.colonnes = C;
    tc.kmax = 0xFFFFFFFFu;  // no partial sums here
    const PrepCodes p = preparer_codes(tc, m);
    if (!p.bon) {  // uniform over the block; counted once here and once by the band kernels
        if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    const trc_disposition disp = disposition(dims_prefill(pp), j);
    uint8_t* mat = reinterpret_cast<uint8_t*>(pp.emplacements + uint64_t(e) * pp.pas_emplacement + disp.base);
    const Avance avance0 = premiere_avance<true>(p, R, g);
    // issued here, ahead of the LDS staging below (which waits on the earlier loads only)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    charge_lut.poser(reinterpret_cast<uint2*>(lds + LDS_LUT));
#pragma unroll
    for (uint32_t k = 0; k < LOT_D; ++k)
        if (k * FILS + threadIdx.x < M / 4u)
            *reinterpret_cast<u32x4*>(lds + LDS_ENT + 16u * (k * FILS + threadIdx.x)) = lutd_v[k];
    if (uniforme32(p.hc.N) == 32u)
        corps_codes_emplacement_n<32>(p, R, mat, mat + disp.echelles, lds, luts + uint64_t(j) * 4u * M, controle,
                                      avance0, g);
    else
        corps_codes_emplacement_n<16>(p, R, mat, mat + disp.echelles, lds, luts + uint64_t(j) * 4u * M, controle,
                                      avance0, g);
}

namespace trc {

// acc[rt] += A_rt x B over the k-steps ks = w, w + 16, ... < B (one 32-value block each) and the
// pieces p < NP of x, for the nrt row tiles of the band, on v_mfma_f32_16x16x32_bf16. Lane g*16 + n
// holds, for A, weights 4g .. 4g + 3 and 16 + 4g .. 19 + 4g of row n of the tile (byte 4g .. 4g + 3
// of its code block, converted with the block's E8M0 scale) and, for B, the same values of x for
// column n: the MFMA adds the products of each lane group's eight K values, so any order common to A
// and B gives the dot product. The B loads of KB k-steps are issued before their MFMAs. Columns past
// the expert's pairs load a valid position; their sums are never stored.
// A batch of B loads: PF_LOT 16-byte loads per lane, KB = PF_LOT / NP k-steps of NP pieces each;
// bq[q * NP + p] is piece p of k-step ks0 + 16 q.
constexpr uint32_t PF_LOT = 6;

// LOT <= PF_LOT: the loads of a batch actually used (KB = LOT / NP k-steps, at least one).
template <uint32_t NP, uint32_t PAS, uint32_t LOT>
__device__ __forceinline__ void charger_b(u32x4 (&bq)[PF_LOT], const uint8_t* xsrc, uint64_t pas_p, uint32_t ks0,
                                          uint32_t B) {
    constexpr uint32_t KB = LOT / NP > 0u ? LOT / NP : 1u;
#pragma unroll
    for (uint32_t q = 0; q < KB; ++q) {
        const uint32_t ks = min(ks0 + PAS * q, B);  // block B of an activation row is zero
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) bq[q * NP + p] = *glob<u32x4>(xsrc + p * pas_p + 64u * ks);
    }
}

template <uint32_t NP, uint32_t NRT, uint32_t PAS, uint32_t LOT>
__device__ __forceinline__ void calculer_b(f32x4 (&acc)[PF_RT_MAX], const u32x4 (&bq)[PF_LOT], uint32_t ks0, uint32_t B,
                                           uint32_t a_codes, uint32_t a_sa, uint32_t lr, uint32_t lg) {
    constexpr uint32_t KB = LOT / NP > 0u ? LOT / NP : 1u;
#pragma unroll
    for (uint32_t q = 0; q < KB; ++q) {
        // straight-line code, so that the B loads stay ahead of every MFMA: a k-step past B
        // multiplies block B - 1 of the weights by the activations' zero block
        const uint32_t ks = min(ks0 + PAS * q, B - 1u);
        bf16x8 a[NRT];
#pragma unroll
        for (uint32_t rt = 0; rt < NRT; ++rt) {
            const uint32_t o = (16u * rt + lr) * B + ks;
            const uint32_t mot = lire_lds<uint32_t>(a_codes + 16u * o + 4u * lg);
            const float sc = __uint_as_float(uint32_t(lire_lds<uint8_t>(a_sa + o)) << 23);
            const bf16x2 p0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(mot, sc, 0);
            const bf16x2 p1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(mot, sc, 1);
            const bf16x2 p2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(mot, sc, 2);
            const bf16x2 p3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(mot, sc, 3);
            a[rt] = bf16x8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
        }
#pragma unroll
        for (uint32_t p = 0; p < NP; ++p) {
            const bf16x8 bv = __builtin_bit_cast(bf16x8, bq[q * NP + p]);
#pragma unroll
            for (uint32_t rt = 0; rt < NRT; ++rt)
                acc[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rt], bv, acc[rt], 0, 0, 0);
        }
    }
}

// The whole product of a column tile over the k-steps w, w + PAS, ...; PRE: the first batch of B is
// already in `pre` (loaded before the band's store, so that its latency hides behind it).
template <uint32_t NP, uint32_t NRT, bool PRE, uint32_t PAS, uint32_t LOT>
__device__ __forceinline__ void produit_bf16(f32x4 (&acc)[PF_RT_MAX], const uint8_t* xsrc, uint64_t pas_p, uint32_t w,
                                             uint32_t B, uint32_t a_codes, uint32_t a_sa, uint32_t lr, uint32_t lg,
                                             const u32x4 (&pre)[PF_LOT]) {
    constexpr uint32_t KB = LOT / NP > 0u ? LOT / NP : 1u;
    uint32_t ks0 = w;
    if constexpr (PRE) {
        if (ks0 < B) {  // wave-uniform
            calculer_b<NP, NRT, PAS, LOT>(acc, pre, ks0, B, a_codes, a_sa, lr, lg);
            ks0 += PAS * KB;
        }
    }
    for (; ks0 < B; ks0 += PAS * KB) {  // wave-uniform
        u32x4 bq[PF_LOT];
        charger_b<NP, PAS, LOT>(bq, xsrc, pas_p, ks0, B);
        __builtin_amdgcn_sched_barrier(0);  // every load issued before the first MFMA waits
        calculer_b<NP, NRT, PAS, LOT>(acc, bq, ks0, B, a_codes, a_sa, lr, lg);
    }
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 15");
    __builtin_amdgcn_sched_barrier(0);
}

// One decode round of a band: the half-wavefront decodes tile t (its lane's 4 code bytes of each
// macro-step kept in registers) and keeps, for lanes v % 4 == 0, the E8M0 byte of its block in each
// macro-step (4 per word), so that the round's entries may be overwritten by the next round.
struct TourBande {
    uint32_t codes[PF_NMAX];
    uint32_t ech[PF_NMAX / 4];
    uint32_t nb;  // macro-steps of the tile (0: no tile)
};

__device__ __forceinline__ void decoder_tour(const EnteteRans& h, const DescFlux& fc, const gptr<u32x4> ent16,
                                             uint32_t t0, uint32_t t_b, uint32_t ba, uint32_t base, TourBande& tb,
                                             uint32_t& hors_l, uint32_t& pointeur) {
    const uint32_t lane = __lane_id();
    const uint32_t v = lane & 31u;
    const bool haut = lane >= 32u;
    const uint32_t decal = haut ? 32u : 0u, masque_inf = (1u << v) - 1u;
    const uint32_t q = v >> 2;
    const uint32_t demi = threadIdx.x >> 5;
    const uint32_t a_lut = base + LDS_LUT;
    const uint32_t a_anneau = base + LDS_ANNEAUX + demi * OCTETS_ANNEAU;
    const uint32_t a_ent = base + LDS_ENT + demi * (ENT_PAR_TUILE * 4u);
    const uint32_t a_ent_q = a_ent + 4u * q;
    const uint32_t N = h.N;
    const uint32_t t = t0 + (haut ? 1u : 0u);
    const bool tuile = t <= t_b;
    const uint32_t nmacro = h.P / 128u;
    const uint32_t nb_a = min(N, nmacro - t0 * N);
    const uint32_t nb_b = t0 + 1u <= t_b ? min(N, nmacro - (t0 + 1u) * N) : 0u;
    const uint32_t nb = haut ? nb_b : nb_a;
    const uint32_t m0 = t * N;
    tb.nb = tuile ? nb : 0u;
    if (tuile) ecrire_lds<u32x4>(a_ent + 16u * v, ent16[2u * m0 + v]);
    uint32_t x = tuile ? h.etats[t * VOIES + v] : L;
    const uint32_t debut = tuile ? h.debut[t] : 0u;
    AnneauR a = ouvrir_anneau_r(h, fc, debut, a_anneau, v, tuile);
    const uint32_t o0 = a.o2;
    uint32_t ent_suiv = tuile ? lire_lds<uint32_t>(a_ent_q) : ENTREE_BOURRAGE;
    const uint32_t nb_min = min(nb_a, nb_b);
    auto macro = [&](auto tous, uint32_t mm) -> uint32_t {
        constexpr bool TOUS = decltype(tous)::value;
        const bool actif = TOUS || mm < nb;
        const uint32_t ent = actif ? ent_suiv : ENTREE_BOURRAGE;
        ent_suiv = lire_lds<uint32_t>(a_ent_q + 32u * ((mm + 1u) & 15u));
        const uint32_t lt = a_lut + (ent & ENT_CTX);
        uint32_t compte = 0;
        const uint32_t e0 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
        const uint32_t e1 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
        const uint32_t e2 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
        const uint32_t e3 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
        a.o2 += 2u * compte;
        avancer_anneau_r(a, v, actif);
        // byte 3 of each LUT word is the decoded byte
        return __builtin_amdgcn_perm(e1, e0, 0x0C0C0703u) | __builtin_amdgcn_perm(e3, e2, 0x07030C0Cu);
    };
#pragma unroll
    for (uint32_t mm = 0; mm < PF_NMAX; ++mm) {
        if (mm < nb_min)
            tb.codes[mm] = macro(std::true_type{}, mm);
        else if (mm < nb_a)
            tb.codes[mm] = macro(std::false_type{}, mm);
        else
            tb.codes[mm] = 0u;
    }
#pragma unroll
    for (uint32_t i = 0; i < PF_NMAX / 4u; ++i) {
        uint32_t w = 0;
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k)
            w |= ((lire_lds<uint32_t>(a_ent_q + 32u * (4u * i + k)) >> ENT_EXP) + 128u & 255u) << (8u * k);
        tb.ech[i] = w;
    }
    // a tile is checked by the band that holds its first block
    if (tuile && m0 * 8u >= ba) {
        hors_l += (x != L) ? 1u : 0u;
        const uint32_t attendu = (t + 1 < h.T) ? h.debut[t + 1] : h.W;
        pointeur += (v == 0 && debut + (a.o2 - o0) / 2u != attendu) ? 1u : 0u;
    }
}

// A round's codes and scales into the band's LDS arrays: codes [row][B][16 B], scales [row][B]. Rows
// hold exactly B blocks, so block beta of the matrix sits at index beta - ba of the band (ba = its
// first block), and no row tracking is needed.
__device__ __forceinline__ void poser_tour(const TourBande& tb, uint32_t t, uint32_t N, uint32_t ba, uint32_t bb,
                                           uint32_t base, uint32_t a_sa) {
    const uint32_t v = __lane_id() & 31u, q = v >> 2;
    const uint32_t beta0 = 8u * t * N + q;
#pragma unroll
    for (uint32_t mm = 0; mm < PF_NMAX; ++mm) {
        const uint32_t beta = beta0 + 8u * mm;
        if (mm < tb.nb && beta >= ba && beta < bb) {
            const uint32_t o = beta - ba;
            ecrire_lds<uint32_t>(base + PF_A + 16u * o + 4u * (v & 3u), tb.codes[mm]);
            if ((v & 3u) == 0u) ecrire_lds<uint8_t>(a_sa + o, uint8_t(tb.ech[mm >> 2] >> (8u * (mm & 3u))));
        }
    }
}

// One band of rows [r0, r0 + nl) of matrix j of expert e against the expert's pairs: its tiles
// decoded in up to two rounds of 32 (one tile per half-wavefront a round), stored in LDS as MXFP4,
// then the bf16 MFMA (weights converted where they are read): each of the 16 waves takes every row
// tile of the band (up to 5) over its share of K, so that each B load feeds every row tile and B is
// read once per band.
template <uint32_t J, bool EMPL>  // EMPL: long tiles, the band copied from the expert's slot
__device__ __forceinline__ void prefill_bande(const ParamsPrefill& pp, const uint32_t* __restrict__ luts,
                                              uint32_t* __restrict__ controle, uint8_t* lds) {
    const uint32_t e = blockIdx.y / J, j = J == 2u ? (blockIdx.y & 1u) : 2u;
    const uint32_t n_e = uniforme32(glob<uint32_t>(reinterpret_cast<const void*>(pp.compte))[e]);
    if (n_e == 0u) return;
    const uint32_t R = choisir(pp.lignes, j), C = choisir(pp.colonnes, j), B = C / 32u;
    const uint32_t RB = choisir(pp.rb, j);
    const uint32_t r0 = blockIdx.x * RB;
    if (r0 >= R) return;
    const uint32_t nl = min(RB, R - r0);
    const uint32_t* lut_src = luts + (uint64_t(j) * 4u + 1u) * M;
    // long tiles: the band's codes and scales come from the expert's slot, nothing is decoded here
    constexpr bool depuis_emplacement = EMPL;
    const uint32_t ba = r0 * B, bb = (r0 + nl) * B;  // the band's blocks
    // the band's blocks [ba, bb) of the slot: 16 code bytes each (16-byte aligned), one scale byte
    // each, read as the 4-byte words of the 256-aligned scale array that cover the band (the vector
    // memory unit takes as long over a byte load as over a 16-byte one). The first batch (PF_LOT_COPIE
    // 16-byte loads and PF_LOT_ECH words per thread: the whole band up to PF_LOT_COPIE * PF_FILS
    // blocks) is requested before anything else, its stores wait until the LDS is free.
    const uint32_t n_copie = nl * B;
    const uint8_t* mat = EMPL ? reinterpret_cast<const uint8_t*>(pp.emplacements + uint64_t(e) * pp.pas_emplacement +
                                                                 disposition(dims_prefill(pp), j).base)
                              : nullptr;
    const gptr<u32x4> codes_c = glob<u32x4>(EMPL ? mat + 16ull * ba : reinterpret_cast<const uint8_t*>(lut_src));
    const gptr<uint32_t> ech32 =
        glob<uint32_t>(EMPL ? mat + disposition(dims_prefill(pp), j).echelles : reinterpret_cast<const uint8_t*>(lut_src));
    const uint32_t w0 = ba >> 2, nw = ((bb + 3u) >> 2) - w0;
    u32x4 c_copie[EMPL ? PF_LOT_COPIE : 1u];
    uint32_t e_copie[EMPL ? PF_LOT_ECH : 1u];
    auto charger_copie = [&](uint32_t i0, uint32_t m0) {
#pragma unroll
        for (uint32_t k = 0; k < PF_LOT_COPIE; ++k) c_copie[k] = codes_c[min(i0 + threadIdx.x + k * PF_FILS, n_copie - 1u)];
#pragma unroll
        for (uint32_t k = 0; k < PF_LOT_ECH; ++k) e_copie[k] = ech32[w0 + min(m0 + threadIdx.x + k * PF_FILS, nw - 1u)];
    };
    if constexpr (EMPL) charger_copie(0u, 0u);
    // the pieces count and the expert's first pair, requested with them (used after the decode)
    const uint32_t p_brut = glob<uint32_t>(reinterpret_cast<const void*>(pp.pieces))[J == 2u ? 0 : 1];
    const uint32_t debut_brut = glob<uint32_t>(reinterpret_cast<const void*>(pp.debut))[e];
    ChargeLut<3> charge_lut;
    if (!depuis_emplacement) charge_lut.demarrer(lut_src, 3u * M / 4u);
    const MatricePartie m = lire_matrice_constante(pp.repertoire + uint64_t(e * 3u + j) * sizeof(MatricePartie));
    const EnteteRans h = entete_de(m.codes, m.cP, m.cN, m.cT, m.cW);
    const uint32_t N = h.N;
    const uint32_t t_a = N ? (ba / 8u) / N : 0u, t_b = N ? ((bb - 1u) / 8u) / N : 0u;
    const bool bon = m.bon != 0u &&
                     (depuis_emplacement || (N >= 1u && N <= PF_NMAX && t_b < h.T && t_b - t_a < 32u * PF_TOURS));
    if (!depuis_emplacement) charge_lut.poser(lut_src, reinterpret_cast<uint2*>(lds + LDS_LUT), 3u * M / 4u);
    // (long tiles: checked once the band is stored, so that the copy's loads are not held back
    // behind the record's)
    if (!depuis_emplacement && !bon) {
        if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    __syncthreads();

    // ---- decode: in round r, half-wavefront h2 of wave w decodes tile t_a + 32 r + 2w + h2
    const uint32_t lane = __lane_id();
    const uint32_t w = threadIdx.x >> 6;
    const uint32_t base = adresse_lds(lds);
    const gptr<u32x4> ent16 = glob<u32x4>(reinterpret_cast<const void*>(pp.ech + uint64_t(e * 3u + j) * pp.pas_ech));
    uint32_t hors_l = 0, pointeur = 0;
    TourBande tour0, tour1;
    tour0.nb = tour1.nb = 0u;
    const uint32_t t00 = t_a + 2u * w, t01 = t00 + 32u;
    // one copy of the decode code for both rounds (a smaller hot loop for the instruction cache)
#pragma nounroll
    for (uint32_t r = 0; r < (depuis_emplacement ? 0u : PF_TOURS); ++r) {
        const uint32_t t0 = r ? t01 : t00;
        TourBande tb;
        tb.nb = 0u;
        if (t0 <= t_b) decoder_tour(h, m.codes, ent16, t0, t_b, ba, base, tb, hors_l, pointeur);
        if (r == 0)
            tour0 = tb;
        else
            tour1 = tb;
    }
    verser_controle(controle, hors_l, pointeur);
    // the first batch of the first column tile's activations is requested now, so that its latency
    // hides behind the store of the codes
    const uint32_t lr = lane & 15u, lg = lane >> 4;
    const uint32_t P = uniforme32(min(p_brut, PF_PIECES_BF));
    const uint32_t debut_e = uniforme32(debut_brut);
    const gptr<uint32_t> paires = glob<uint32_t>(reinterpret_cast<const void*>(pp.paires));
    const uint64_t pas_p = uint64_t(J == 2u ? pp.bx : pp.bact) * 64u;
    const uint8_t* bsrc = reinterpret_cast<const uint8_t*>(J == 2u ? pp.xb : pp.ab) + 16u * lg;
    const uint32_t wu = uniforme32(w);
    // Column tiles of 16 pairs go two at a time while two remain, waves 0-7 on the first and 8-15
    // on the second (K split 8 ways), then one at a time (K split 16 ways).
    const uint32_t n_tt = (n_e + 15u) / 16u;
    const bool duo0 = n_tt >= 2u;
    // the first pass's tile and K share of this wave, and its column
    const uint32_t g0 = duo0 ? wu >> 3 : 0u, wk0 = duo0 ? (wu & 7u) : wu;
    const uint32_t tok0 = 16u * g0 + lr;
    const uint32_t c0 = tok0 < n_e ? paires[debut_e + tok0] : paires[debut_e];
    // loads per B batch: six for gate/up (x: one piece), three for down (act: three pieces), which
    // measured faster there than six
    constexpr uint32_t LOT = J == 2u ? PF_LOT : 3u;
    u32x4 pre[PF_LOT];
    {
        const uint8_t* src0 = bsrc + uint64_t(J == 2u ? c0 / pp.k : c0) * PF_PIECES_BF * pas_p;
        auto charger0 = [&](auto np) {
            constexpr uint32_t NP = decltype(np)::value;
            if (duo0)
                charger_b<NP, 8, LOT>(pre, src0, pas_p, wk0, B);
            else
                charger_b<NP, 16, LOT>(pre, src0, pas_p, wk0, B);
        };
        using U = uint32_t;
        if (wk0 < B) {  // wave-uniform
            if (P == 1u)
                charger0(std::integral_constant<U, 1>{});
            else if (P == 2u)
                charger0(std::integral_constant<U, 2>{});
            else if (P == 3u)
                charger0(std::integral_constant<U, 3>{});
        }
    }
    __syncthreads();  // every tile decoded: the LUT, x and ring regions are free

    // ---- store the band's codes and scales
    const uint32_t a_sa = base + pf_sa(RB, B), a_part = base + pf_part(RB, B);
    const uint32_t haut = lane >= 32u ? 1u : 0u;
    if constexpr (EMPL) {
        for (uint32_t i0 = 0, m0 = 0; i0 < n_copie; i0 += PF_LOT_COPIE * PF_FILS, m0 += PF_LOT_ECH * PF_FILS) {
            if (i0 > 0u) charger_copie(i0, m0);  // bands past one batch
#pragma unroll
            for (uint32_t k = 0; k < PF_LOT_COPIE; ++k) {
                const uint32_t i = i0 + threadIdx.x + k * PF_FILS;
                if (i < n_copie) ecrire_lds<u32x4>(base + PF_A + 16u * i, c_copie[k]);
            }
#pragma unroll
            for (uint32_t k = 0; k < PF_LOT_ECH; ++k) {
                const uint32_t i = m0 + threadIdx.x + k * PF_FILS;
#pragma unroll
                for (uint32_t o = 0; o < 4u; ++o) {
                    const uint32_t blk = 4u * (w0 + i) + o;
                    if (i < nw && blk >= ba && blk < bb) ecrire_lds<uint8_t>(a_sa + blk - ba, uint8_t(e_copie[k] >> (8u * o)));
                }
            }
        }
    } else {
        poser_tour(tour0, t00 + haut, N, ba, bb, base, a_sa);
        poser_tour(tour1, t01 + haut, N, ba, bb, base, a_sa);
    }
    if (depuis_emplacement && !bon) {  // uniform over the block
        if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    // padding: rows nl .. RB - 1 of a last, partial band (zero codes, scale 1)
    for (uint32_t i = threadIdx.x; i < (RB - nl) * B; i += blockDim.x) {
        const uint32_t o = nl * B + i;
        ecrire_lds<u32x4>(base + PF_A + 16u * o, u32x4{0u, 0u, 0u, 0u});
        ecrire_lds<uint8_t>(a_sa + o, uint8_t(ECHELLE_UN));
    }
    __syncthreads();

    // ---- MFMA: every wave takes all nrt row tiles and the k-steps (blocks) ks = w, w + 16, ..., K
    // split 16 ways; the partial sums are added in wave order. Each B load feeds every row tile, and
    // B is read once per band.
    const uint32_t nrt = RB / 16u;
    const gptr<float> biais = glob<float>(reinterpret_cast<const void*>(m.biais.p));
    // one pass over NT column tiles from tile tt; the first pass is peeled off the loop so that its
    // preloaded B dies there
    auto passe = [&](uint32_t tt, auto nt_t, auto premier) {
        constexpr uint32_t NT = decltype(nt_t)::value;
        constexpr bool PREMIER = decltype(premier)::value;
        constexpr uint32_t PAS = 16u / NT, VG = 16u / NT;  // waves per tile
        const uint32_t g = NT == 2u ? wu >> 3 : 0u, wk = NT == 2u ? (wu & 7u) : wu;
        const uint32_t tok = 16u * (tt + g) + lr;
        const uint32_t c = PREMIER ? c0 : (tok < n_e ? paires[debut_e + tok] : paires[debut_e]);
        // column source: position c / k's x for gate and up, pair c's act for down
        const uint8_t* src = bsrc + uint64_t(J == 2u ? c / pp.k : c) * PF_PIECES_BF * pas_p;
        f32x4 acc[PF_RT_MAX];
#pragma unroll
        for (uint32_t rt = 0; rt < PF_RT_MAX; ++rt) acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto produit = [&](auto np) {
            constexpr uint32_t NP = decltype(np)::value;
            if (nrt == 5u)
                produit_bf16<NP, 5, PREMIER, PAS, LOT>(acc, src, pas_p, wk, B, base + PF_A, a_sa, lr, lg, pre);
            else if (nrt == 4u)
                produit_bf16<NP, 4, PREMIER, PAS, LOT>(acc, src, pas_p, wk, B, base + PF_A, a_sa, lr, lg, pre);
            else if (nrt == 2u)
                produit_bf16<NP, 2, PREMIER, PAS, LOT>(acc, src, pas_p, wk, B, base + PF_A, a_sa, lr, lg, pre);
            else
                produit_bf16<NP, 1, PREMIER, PAS, LOT>(acc, src, pas_p, wk, B, base + PF_A, a_sa, lr, lg, pre);
        };
        using U = uint32_t;
        if (P == 1u)
            produit(std::integral_constant<U, 1>{});
        else if (P == 2u)
            produit(std::integral_constant<U, 2>{});
        else if (P == 3u)
            produit(std::integral_constant<U, 3>{});
        // partial sums: [tile g][row tile][wave of the tile's first half][lane], nrt x 8 KiB for either
        // pass shape. The second half of a tile's waves stores its sums, the first half adds them to
        // its own (wave wk + MI to wave wk) and stores the results, which are added in wave order.
        constexpr uint32_t MI = VG / 2u;
        const bool second = wk >= MI;
        const uint32_t wl = second ? wk - MI : wk;
        const uint32_t a_moi = a_part + ((g * nrt * MI + wl) * 64u + lane) * 16u;  // row tile rt: + rt MI KiB
        if (second) {
#pragma unroll
            for (uint32_t rt = 0; rt < PF_RT_MAX; ++rt)
                if (rt < nrt) ecrire_lds<f32x4>(a_moi + rt * MI * 1024u, acc[rt]);
        }
        __syncthreads();
        if (!second) {
#pragma unroll
            for (uint32_t rt = 0; rt < PF_RT_MAX; ++rt)
                if (rt < nrt) {
                    const f32x4 autre = lire_lds<f32x4>(a_moi + rt * MI * 1024u);
                    ecrire_lds<f32x4>(a_moi + rt * MI * 1024u, acc[rt] + autre);
                }
        }
        __syncthreads();
        constexpr uint32_t TOURS_SOMME = (NT * PF_RT_MAX * 256u + 1023u) / 1024u;
#pragma unroll
        for (uint32_t u = 0; u < TOURS_SOMME; ++u) {
            const uint32_t o = threadIdx.x + 1024u * u;  // output (tile gg, row tile, column, row)
            const uint32_t gg = NT == 2u ? o / (nrt * 256u) : 0u, reste_o = o - gg * (nrt * 256u);
            if (gg < NT && reste_o < nrt * 256u) {
                const uint32_t rt = reste_o >> 8, reste = reste_o & 255u;
                const uint32_t ln = reste >> 2, r = reste & 3u;
                float s = 0.0f;
                for (uint32_t ww = 0; ww < MI; ++ww)
                    s += lire_lds<float>(a_part + (((gg * nrt + rt) * MI + ww) * 64u + ln) * 16u + 4u * r);
                const uint32_t ligne = 16u * rt + 4u * (ln >> 4) + r, jeton = 16u * (tt + gg) + (ln & 15u);
                if (ligne < nl && jeton < n_e) {
                    const uint32_t cc = paires[debut_e + jeton];
                    const float y = s + biais[r0 + ligne];
                    if (J == 2u)
                        ecrire_global<float>(reinterpret_cast<float*>(pp.gu) + (uint64_t(cc) * 2u + j) * R + r0 + ligne, y);
                    else
                        ecrire_global<float>(reinterpret_cast<float*>(pp.s) + uint64_t(cc) * pp.D + r0 + ligne, y);
                }
            }
        }
        __syncthreads();
    };
    using U2 = uint32_t;
    uint32_t tt = 0;
    if (duo0) {
        passe(0u, std::integral_constant<U2, 2>{}, std::true_type{});
        tt = 2u;
    } else {
        passe(0u, std::integral_constant<U2, 1>{}, std::true_type{});  // n_e >= 1
        tt = 1u;
    }
    for (; tt + 1u < n_tt; tt += 2u) passe(tt, std::integral_constant<U2, 2>{}, std::false_type{});
    if (tt < n_tt) passe(tt, std::integral_constant<U2, 1>{}, std::false_type{});
}

// ------------------------------------------------- band kernels over the slots, two blocks per CU
// Long tiles: every chosen expert sits decoded in its slot, so a band is a copy (one batch of loads,
// issued first), then the MFMA passes. A block holds one band of PFE_RB rows with PFE_FILS threads
// in under half the LDS, so that two blocks share a CU and one's copy and prologue run under the
// other's MFMA passes and reductions. Same operands, k-steps and pass shapes as prefill_bande, with
// 8 wavefronts: one column tile at a time splits K 8 ways, two at a time 4 ways each. Used for gate
// and up (x: one bf16 piece); down, whose act has three pieces, reads 2.5 times the activation bytes
// over bands of 32 rows and measured faster with prefill_bande's bands of 80 (289 against 407 us for
// config 5, gate/up 433 against 463 us).
constexpr uint32_t PFE_FILS = 512;
constexpr uint32_t PFE_RB = 32;                  // rows per band: 2 row tiles
constexpr uint32_t PFE_NRT = PFE_RB / 16u;
constexpr uint32_t PFE_LOT = 8;                  // 16-byte code loads per thread: 4096 blocks a batch
constexpr uint32_t PFE_LOT_ECH = PFE_LOT / 4u;   // scale words with them
constexpr uint32_t PFE_PART = PFE_NRT * 4u * 64u * 16u;  // partial sums: row tiles x 4 waves x 64 lanes x 16 B
constexpr uint32_t PFE_LDS = PFE_RB * PF_BP_MAX * 16u + PFE_RB * PF_BP_MAX + PFE_PART;
static_assert(PFE_LDS <= LDS_GEMV / 2u, "two blocks per CU");

template <uint32_t J>
__device__ __forceinline__ void prefill_bande_empl(const ParamsPrefill& pp, uint32_t* __restrict__ controle, uint8_t* lds) {
    constexpr uint32_t FILS = PFE_FILS, NRT = PFE_NRT, RB = PFE_RB;
    const uint32_t e = blockIdx.y / J, j = J == 2u ? (blockIdx.y & 1u) : 2u;
    const uint32_t n_e = uniforme32(glob<uint32_t>(reinterpret_cast<const void*>(pp.compte))[e]);
    if (n_e == 0u) return;
    const uint32_t R = choisir(pp.lignes, j), C = choisir(pp.colonnes, j), B = C / 32u;
    const uint32_t r0 = blockIdx.x * RB;
    if (r0 >= R) return;
    const uint32_t nl = min(RB, R - r0);
    const uint32_t ba = r0 * B, bb = (r0 + nl) * B;  // the band's blocks
    // the band's blocks [ba, bb) of the slot (16 code bytes each) and the 4-byte words of the scale
    // array that cover them, requested before anything else; stored once the pass is set up
    const uint32_t n = nl * B;
    const trc_disposition disp = disposition(dims_prefill(pp), j);
    const uint8_t* mat = reinterpret_cast<const uint8_t*>(pp.emplacements + uint64_t(e) * pp.pas_emplacement + disp.base);
    const gptr<u32x4> codes = glob<u32x4>(mat + 16ull * ba);
    const gptr<uint32_t> ech32 = glob<uint32_t>(mat + disp.echelles);
    const uint32_t w0 = ba >> 2, nw = ((bb + 3u) >> 2) - w0;
    u32x4 c[PFE_LOT];
    uint32_t e4[PFE_LOT_ECH];
    auto charger_copie = [&](uint32_t i0, uint32_t m0) {
#pragma unroll
        for (uint32_t k = 0; k < PFE_LOT; ++k) c[k] = codes[min(i0 + threadIdx.x + k * FILS, n - 1u)];
#pragma unroll
        for (uint32_t k = 0; k < PFE_LOT_ECH; ++k) e4[k] = ech32[w0 + min(m0 + threadIdx.x + k * FILS, nw - 1u)];
    };
    charger_copie(0u, 0u);
    const uint32_t p_brut = glob<uint32_t>(reinterpret_cast<const void*>(pp.pieces))[J == 2u ? 0 : 1];
    const uint32_t debut_brut = glob<uint32_t>(reinterpret_cast<const void*>(pp.debut))[e];
    const MatricePartie m = lire_matrice_constante(pp.repertoire + uint64_t(e * 3u + j) * sizeof(MatricePartie));
    const uint32_t lane = __lane_id(), lr = lane & 15u, lg = lane >> 4;
    const uint32_t wu = uniforme32(threadIdx.x >> 6);
    const uint32_t base = adresse_lds(lds);
    const uint32_t P = uniforme32(min(p_brut, PF_PIECES_BF));
    const uint32_t debut_e = uniforme32(debut_brut);
    const gptr<uint32_t> paires = glob<uint32_t>(reinterpret_cast<const void*>(pp.paires));
    const uint64_t pas_p = uint64_t(J == 2u ? pp.bx : pp.bact) * 64u;
    const uint8_t* bsrc = reinterpret_cast<const uint8_t*>(J == 2u ? pp.xb : pp.ab) + 16u * lg;
    // Column tiles of 16 pairs go two at a time while two remain, waves 0-3 on the first and 4-7 on
    // the second (K split 4 ways), then one at a time (K split 8 ways). The first batch of the first
    // pass's activations is requested before the band is stored.
    const uint32_t n_tt = (n_e + 15u) / 16u;
    const bool duo0 = n_tt >= 2u;
    const uint32_t g0 = duo0 ? wu >> 2 : 0u, wk0 = duo0 ? (wu & 3u) : wu;
    const uint32_t tok0 = 16u * g0 + lr;
    const uint32_t c0 = tok0 < n_e ? paires[debut_e + tok0] : paires[debut_e];
    constexpr uint32_t LOT = J == 2u ? PF_LOT : 3u;
    u32x4 pre[PF_LOT];
    {
        const uint8_t* src0 = bsrc + uint64_t(J == 2u ? c0 / pp.k : c0) * PF_PIECES_BF * pas_p;
        auto charger0 = [&](auto np) {
            constexpr uint32_t NP = decltype(np)::value;
            if (duo0)
                charger_b<NP, 4, LOT>(pre, src0, pas_p, wk0, B);
            else
                charger_b<NP, 8, LOT>(pre, src0, pas_p, wk0, B);
        };
        using U = uint32_t;
        if (wk0 < B) {  // wave-uniform
            if (P == 1u)
                charger0(std::integral_constant<U, 1>{});
            else if (P == 2u)
                charger0(std::integral_constant<U, 2>{});
            else if (P == 3u)
                charger0(std::integral_constant<U, 3>{});
        }
    }
    // ---- the band into LDS: codes [row][B][16 B], scales [row][B], zero padding rows
    const uint32_t a_sa = base + pf_sa(RB, B), a_part = base + pf_part(RB, B);
    for (uint32_t i0 = 0, m0 = 0; i0 < n || m0 < nw; i0 += PFE_LOT * FILS, m0 += PFE_LOT_ECH * FILS) {
        if (i0 > 0u) charger_copie(i0, m0);  // bands past one batch
#pragma unroll
        for (uint32_t k = 0; k < PFE_LOT; ++k) {
            const uint32_t i = i0 + threadIdx.x + k * FILS;
            if (i < n) ecrire_lds<u32x4>(base + PF_A + 16u * i, c[k]);
        }
#pragma unroll
        for (uint32_t k = 0; k < PFE_LOT_ECH; ++k) {
            const uint32_t i = m0 + threadIdx.x + k * FILS;
#pragma unroll
            for (uint32_t o = 0; o < 4u; ++o) {
                const uint32_t blk = 4u * (w0 + i) + o;
                if (i < nw && blk >= ba && blk < bb) ecrire_lds<uint8_t>(a_sa + blk - ba, uint8_t(e4[k] >> (8u * o)));
            }
        }
    }
    if (m.bon == 0u) {  // uniform over the block; checked after the copy so that its loads go first
        if (blockIdx.x == 0 && threadIdx.x == 0) atomicAdd(&controle[CTL_FORMAT], 1u);
        return;
    }
    for (uint32_t i = threadIdx.x; i < (RB - nl) * B; i += FILS) {
        const uint32_t o = nl * B + i;
        ecrire_lds<u32x4>(base + PF_A + 16u * o, u32x4{0u, 0u, 0u, 0u});
        ecrire_lds<uint8_t>(a_sa + o, uint8_t(ECHELLE_UN));
    }
    __syncthreads();

    // ---- MFMA passes (as prefill_bande's, 8 wavefronts)
    const gptr<float> biais = glob<float>(reinterpret_cast<const void*>(m.biais.p));
    auto passe = [&](uint32_t tt, auto nt_t, auto premier) {
        constexpr uint32_t NT = decltype(nt_t)::value;
        constexpr bool PREMIER = decltype(premier)::value;
        constexpr uint32_t PAS = 8u / NT, VG = 8u / NT;  // waves per tile
        const uint32_t g = NT == 2u ? wu >> 2 : 0u, wk = NT == 2u ? (wu & 3u) : wu;
        const uint32_t tok = 16u * (tt + g) + lr;
        const uint32_t cl = PREMIER ? c0 : (tok < n_e ? paires[debut_e + tok] : paires[debut_e]);
        const uint8_t* src = bsrc + uint64_t(J == 2u ? cl / pp.k : cl) * PF_PIECES_BF * pas_p;
        f32x4 acc[PF_RT_MAX];
#pragma unroll
        for (uint32_t rt = 0; rt < PF_RT_MAX; ++rt) acc[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto produit = [&](auto np) {
            constexpr uint32_t NP = decltype(np)::value;
            produit_bf16<NP, NRT, PREMIER, PAS, LOT>(acc, src, pas_p, wk, B, base + PF_A, a_sa, lr, lg, pre);
        };
        using U = uint32_t;
        if (P == 1u)
            produit(std::integral_constant<U, 1>{});
        else if (P == 2u)
            produit(std::integral_constant<U, 2>{});
        else if (P == 3u)
            produit(std::integral_constant<U, 3>{});
        // partial sums: [tile g][row tile][wave of the tile's first half][lane]. The second half of a
        // tile's waves stores its sums, the first half adds them to its own and stores the results,
        // which are added in wave order.
        constexpr uint32_t MI = VG / 2u;
        const bool second = wk >= MI;
        const uint32_t wl = second ? wk - MI : wk;
        const uint32_t a_moi = a_part + ((g * NRT * MI + wl) * 64u + lane) * 16u;  // row tile rt: + rt MI KiB
        if (second) {
#pragma unroll
            for (uint32_t rt = 0; rt < NRT; ++rt) ecrire_lds<f32x4>(a_moi + rt * MI * 1024u, acc[rt]);
        }
        __syncthreads();
        if (!second) {
#pragma unroll
            for (uint32_t rt = 0; rt < NRT; ++rt) {
                const f32x4 autre = lire_lds<f32x4>(a_moi + rt * MI * 1024u);
                ecrire_lds<f32x4>(a_moi + rt * MI * 1024u, acc[rt] + autre);
            }
        }
        __syncthreads();
        constexpr uint32_t TOURS_SOMME = (NT * NRT * 256u + FILS - 1u) / FILS;
#pragma unroll
        for (uint32_t u = 0; u < TOURS_SOMME; ++u) {
            const uint32_t o = threadIdx.x + FILS * u;  // output (tile gg, row tile, column, row)
            const uint32_t gg = NT == 2u ? o / (NRT * 256u) : 0u, reste_o = o - gg * (NRT * 256u);
            if (gg < NT && reste_o < NRT * 256u) {
                const uint32_t rt = reste_o >> 8, reste = reste_o & 255u;
                const uint32_t ln = reste >> 2, r = reste & 3u;
                float s = 0.0f;
                for (uint32_t ww = 0; ww < MI; ++ww)
                    s += lire_lds<float>(a_part + (((gg * NRT + rt) * MI + ww) * 64u + ln) * 16u + 4u * r);
                const uint32_t ligne = 16u * rt + 4u * (ln >> 4) + r, jeton = 16u * (tt + gg) + (ln & 15u);
                if (ligne < nl && jeton < n_e) {
                    const uint32_t cc = paires[debut_e + jeton];
                    const float y = s + biais[r0 + ligne];
                    if (J == 2u)
                        ecrire_global<float>(reinterpret_cast<float*>(pp.gu) + (uint64_t(cc) * 2u + j) * R + r0 + ligne, y);
                    else
                        ecrire_global<float>(reinterpret_cast<float*>(pp.s) + uint64_t(cc) * pp.D + r0 + ligne, y);
                }
            }
        }
        __syncthreads();
    };
    using U2 = uint32_t;
    uint32_t tt = 0;
    if (duo0) {
        passe(0u, std::integral_constant<U2, 2>{}, std::true_type{});
        tt = 2u;
    } else {
        passe(0u, std::integral_constant<U2, 1>{}, std::true_type{});  // n_e >= 1
        tt = 1u;
    }
    for (; tt + 1u < n_tt; tt += 2u) passe(tt, std::integral_constant<U2, 2>{}, std::false_type{});
    if (tt < n_tt) passe(tt, std::integral_constant<U2, 1>{}, std::false_type{});
}

}  // namespace trc

extern "C" __global__ void __launch_bounds__(trc::PFE_FILS) __attribute__((amdgpu_waves_per_eu(4)))
prefill_bande_gu_emplacement(ParamsPrefill pp, uint32_t* __restrict__ controle) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[trc::PFE_LDS];
    trc::prefill_bande_empl<2>(pp, controle, lds);
}

extern "C" __global__ void __launch_bounds__(trc::PF_FILS)
prefill_mfma_gu(ParamsPrefill pp, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    __shared__ __attribute__((aligned(16384))) uint8_t lds[trc::LDS_GEMV];
    trc::prefill_bande<2, false>(pp, luts, controle, lds);
}

extern "C" __global__ void __launch_bounds__(trc::PF_FILS)
prefill_mfma_bas(ParamsPrefill pp, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    __shared__ __attribute__((aligned(16384))) uint8_t lds[trc::LDS_GEMV];
    trc::prefill_bande<1, false>(pp, luts, controle, lds);
}

// Down over long tiles: each band copied from its expert's slot (gate and up take
// prefill_bande_gu_emplacement).
extern "C" __global__ void __launch_bounds__(trc::PF_FILS)
prefill_mfma_bas_emplacement(ParamsPrefill pp, const uint32_t* __restrict__ luts, uint32_t* __restrict__ controle) {
    __shared__ __attribute__((aligned(16384))) uint8_t lds[trc::LDS_GEMV];
    trc::prefill_bande<1, true>(pp, luts, controle, lds);
}

// x_i[r] += ((w0 s_i0[r] + w1 s_i1[r]) + w2 s_i2[r]) + ..., each product and sum rounded on its own
// (combiner_pos, trc-modele/src/lib.rs:706-710 -> passe.cuh:611-622); positions whose experts are
// not all valid, mounted matrices are left alone. A thread takes 4 consecutive rows when pp.quatre
// (16-byte loads and stores), else one.
extern "C" __global__ void __launch_bounds__(256)
prefill_combiner(ParamsPrefill pp) {
#pragma clang fp contract(off)
    using namespace trc;
    const uint32_t i = blockIdx.y, g = blockIdx.x * 256u + threadIdx.x;
    const uint32_t k = pp.k, D = pp.D;
    const bool quatre = pp.quatre != 0u;
    const uint32_t r = quatre ? 4u * g : g;
    if (r >= D) return;
    const uint32_t* idx = reinterpret_cast<const uint32_t*>(pp.indices) + uint64_t(i) * k;
    bool ok = true;
    for (uint32_t s = 0; s < k; ++s) {
        const uint32_t e = idx[s];
        ok = ok && e < pp.E;
        if (ok)
            for (uint32_t j = 0; j < 3; ++j)
                ok = ok && reinterpret_cast<const MatricePartie*>(pp.repertoire)[e * 3u + j].bon != 0u;
    }
    if (!ok) return;
    const float* w = reinterpret_cast<const float*>(pp.poids) + uint64_t(i) * k;
    const float* s = reinterpret_cast<const float*>(pp.s) + uint64_t(i) * k * D;
    float* x = reinterpret_cast<float*>(pp.residus) + uint64_t(i) * D;
    if (quatre) {
        const float w0 = w[0];
        f32x4 v = *reinterpret_cast<const f32x4*>(s + r);
        f32x4 acc = {w0 * v.x, w0 * v.y, w0 * v.z, w0 * v.w};
        for (uint32_t q = 1; q < k; ++q) {
            const float wq = w[q];
            v = *reinterpret_cast<const f32x4*>(s + uint64_t(q) * D + r);
            const f32x4 p = {wq * v.x, wq * v.y, wq * v.z, wq * v.w};
            acc = f32x4{acc.x + p.x, acc.y + p.y, acc.z + p.z, acc.w + p.w};
        }
        f32x4 xr = *reinterpret_cast<const f32x4*>(x + r);
        xr = f32x4{xr.x + acc.x, xr.y + acc.y, xr.z + acc.z, xr.w + acc.w};
        *reinterpret_cast<f32x4*>(x + r) = xr;
    } else {
        float acc = w[0] * s[r];
        for (uint32_t q = 1; q < k; ++q) {
            const float p = w[q] * s[uint64_t(q) * D + r];
            acc = acc + p;
        }
        x[r] = x[r] + acc;
    }
}

// ============================================================================ C-ABI launch layer
namespace trc {
int lancer_echelles_prefill(const ParamsMoe& pm, uint32_t R, uint32_t C, uint32_t n_delta, const uint32_t* luts,
                            uint32_t* ctl, hipStream_t f);
uint64_t octets_entrees(uint32_t R, uint32_t C);
}  // namespace trc

namespace {

using trc::usage;

uint64_t al(uint64_t x) { return (x + 255u) & ~uint64_t(255); }

// Rows per band: 80, 64, 32 or 16, the most whose CODES_CTX tiles (N macro-steps of 8 blocks each)
// fit the 64 tiles a block decodes in two rounds and whose codes, scales and partial sums fit the LDS;
// 0 if none does. The more of the 64 tile slots a band fills, the fewer wavefronts idle in the second
// round (gpt-oss rows: 80 rows are 56.25 tiles, 64 rows 45).
// Tiles of 16 macro-steps or more (bands copied from the slots, nothing decoded per band): the LDS
// alone decides.
bool tuiles_longues(uint32_t N) { return N >= trc::PF_NMAX; }

uint32_t rb_de(uint32_t B, uint32_t N) {
    for (const uint32_t rb : {trc::PF_RB_MAX, 64u, 32u, 16u})
        if ((tuiles_longues(N) || (rb * B - 1u) / (8u * N) + 2u <= 32u * trc::PF_TOURS) && trc::pf_lds_tient(rb, B))
            return rb;
    return 0;
}

struct Disposition {
    uint64_t pieces, compte, debut, paires, ech, pas_ech, xb, gu, ab, s, emplacements, pas_emplacement, total;
};

int disposer(const trc_dims_expert* dims, uint32_t E, uint32_t T, uint32_t k, uint32_t n_codes, Disposition& d) {
    if (dims == nullptr) return usage("dims absent");
    int r = trc_dims_verifier(dims);
    if (r != TRC_OK) return r;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0], D = dims->lignes[2];
    if (dims->lignes[1] != R || dims->colonnes[1] != C || dims->colonnes[2] != R)
        return usage("gate, up et down incompatibles");
    if (D != C) return usage("la sortie des experts (%u) doit avoir la taille de x (%u)", D, C);
    if (C > 32u * trc::PF_BP_MAX || R > 32u * trc::PF_BP_MAX)
        return usage("prefill : au plus %u colonnes (%u x %u)", 32u * trc::PF_BP_MAX, R, C);
    for (int j = 0; j < 3; ++j)
        if (dims->colonnes[j] / 32 < 8) return usage("matrice %d : moins de 8 blocs par ligne", j);
    if (n_codes == 0 || n_codes > 65535) return usage("prefill : N de CODES_CTX %u", n_codes);
    for (int j = 0; j < 3; ++j)
        if (rb_de(dims->colonnes[j] / 32, n_codes) == 0) return usage("prefill : N = %u trop petit", n_codes);
    if (E == 0 || E > trc::EXPERTS_MAX || k == 0 || k > trc::TOPK_MAX || k > E) return usage("top-%u sur %u", k, E);
    if (T == 0 || uint64_t(T) * k > trc::PF_PAIRES_MAX)
        return usage("prefill : %u positions x %u (au plus %u paires)", T, k, trc::PF_PAIRES_MAX);
    const uint32_t Rm = D > R ? D : R;
    const uint64_t n = uint64_t(T) * k;
    uint64_t p = 0;
    d.pieces = p;
    p += al(16);
    d.compte = p;
    p += al(4ull * E);
    d.debut = p;
    p += al(4ull * E);
    d.paires = p;
    p += al(4ull * n);
    d.pas_ech = 0;
    d.ech = 0;
    d.emplacements = 0;
    d.pas_emplacement = 0;
    if (tuiles_longues(n_codes)) {  // one slot per expert of the layer (the chosen ones are decoded)
        d.pas_emplacement = trc_taille_emplacement(dims);
        d.emplacements = p;
        p += uint64_t(E) * d.pas_emplacement;
    } else {  // the DELTA pass's block entries
        d.pas_ech = trc::octets_entrees(Rm, C);
        d.ech = p;
        p += 3ull * E * d.pas_ech;
    }
    d.xb = p;
    p += al(64ull * T * trc::PF_PIECES_BF * (C / 32u + 1u));
    d.gu = p;
    p += al(4ull * n * 2u * R);
    d.ab = p;
    p += al(64ull * n * trc::PF_PIECES_BF * (R / 32u + 1u));
    d.s = p;
    p += al(4ull * n * D);
    d.total = p;
    return TRC_OK;
}

}  // namespace

extern "C" uint64_t trc_taille_travail_prefill(const trc_dims_expert* dims, uint32_t experts, uint32_t positions,
                                               uint32_t k, uint32_t n_codes) {
    Disposition d;
    if (disposer(dims, experts, positions, k, n_codes, d) != TRC_OK) return 0;
    return d.total;
}

// Config 5: batched prefill of one resident MoE layer. For each position i < T, slot q < k:
// s_iq = W_down swiglu(W_gate x_i + b_gate, W_up x_i + b_up) + b_down of expert indices[i*k + q],
// then residus_i += ((w_i0 s_i0 + w_i1 s_i1) + ...). Each chosen expert is decoded once, by bands of
// rows, and applied to all its positions on the MFMA. No host sync.
extern "C" int trc_prefill_moe(trc_vue repertoire, uint32_t experts, trc_vue luts, const trc_dims_expert* dims,
                               trc_vue x, uint32_t positions, trc_vue indices, trc_vue poids, uint32_t k,
                               trc_vue residus, trc_vue controle, trc_vue travail, uint32_t n_delta,
                               uint32_t n_codes, void* flux) {
    Disposition d;
    int r = disposer(dims, experts, positions, k, n_codes, d);
    if (r != TRC_OK) return r;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0], D = dims->lignes[2], T = positions;
    TRC_VERIFIER(n_delta > 0 && n_delta <= 65535, "N de DELTA %u", n_delta);
    TRC_VERIFIER(repertoire.adresse && repertoire.octets >= 3ull * experts * sizeof(trc::MatricePartie) &&
                     repertoire.adresse % 16 == 0,
                 "repertoire trop court ou non aligne sur 16");
    TRC_VERIFIER(luts.adresse && luts.octets >= uint64_t(trc::LUTS_PAR_COUCHE) * 4, "LUT trop courtes");
    TRC_VERIFIER(x.adresse && x.octets >= 4ull * T * C && x.adresse % 16 == 0, "x trop court ou non aligne");
    TRC_VERIFIER(indices.adresse && indices.octets >= 4ull * T * k && poids.adresse && poids.octets >= 4ull * T * k,
                 "indices ou poids trop courts");
    TRC_VERIFIER(residus.adresse && residus.octets >= 4ull * T * D, "residus trop courts");
    TRC_VERIFIER(controle.adresse && controle.octets >= 16, "controle de moins de 16 o");
    TRC_VERIFIER(travail.adresse && travail.octets >= d.total && travail.adresse % 256 == 0,
                 "travail de %llu o, %llu o demandes (aligne sur 256)", (unsigned long long)travail.octets,
                 (unsigned long long)d.total);
    const uint64_t b = travail.adresse;
    ParamsPrefill pp;
    std::memset(&pp, 0, sizeof(pp));
    pp.repertoire = repertoire.adresse;
    pp.ech = b + d.ech;
    pp.pas_ech = d.pas_ech;
    pp.compte = b + d.compte;
    pp.debut = b + d.debut;
    pp.paires = b + d.paires;
    pp.pieces = b + d.pieces;
    pp.indices = indices.adresse;
    pp.poids = poids.adresse;
    pp.x = x.adresse;
    pp.residus = residus.adresse;
    pp.emplacements = d.pas_emplacement ? b + d.emplacements : 0u;
    pp.pas_emplacement = d.pas_emplacement;
    pp.xb = b + d.xb;
    pp.gu = b + d.gu;
    pp.ab = b + d.ab;
    pp.s = b + d.s;
    for (int j = 0; j < 3; ++j) {
        pp.lignes[j] = dims->lignes[j];
        pp.colonnes[j] = dims->colonnes[j];
        pp.rb[j] = rb_de(dims->colonnes[j] / 32, n_codes);
    }
    pp.T = T;
    pp.bx = C / 32u + 1u;
    pp.bact = R / 32u + 1u;
    pp.quatre = (D % 4u == 0u && residus.adresse % 16u == 0u) ? 1u : 0u;
    pp.k = k;
    pp.E = experts;
    pp.D = D;

    trc::ParamsMoe pm;
    std::memset(&pm, 0, sizeof(pm));
    pm.repertoire = repertoire.adresse;
    pm.ech = pp.ech;
    pm.pas = d.pas_ech;
    pm.compte = pp.compte;
    pm.k = k;
    pm.E = experts;
    for (int j = 0; j < 3; ++j) {
        pm.lignes[j] = dims->lignes[j];
        pm.colonnes[j] = dims->colonnes[j];
    }
    const hipStream_t f = reinterpret_cast<hipStream_t>(flux);
    auto ctl = reinterpret_cast<uint32_t*>(controle.adresse);
    const uint32_t* l = reinterpret_cast<const uint32_t*>(luts.adresse);
    const uint32_t Rm = D > R ? D : R;
    TRC_LANCER(prefill_grouper, dim3(1), dim3(1024), f, pp, ctl);
    TRC_LANCER(prefill_quant_x, dim3(T), dim3(trc::PF_Q_FILS), f, pp);
    if (pp.emplacements != 0 && trc::delta_dans_codes(n_delta, n_codes)) {
        // every chosen expert decoded once into its slot, each tile's DELTA with it:
        // PF_PAIRES_RAPIDE tile pairs per wavefront over the largest of the three matrices
        uint32_t tc = 1;
        for (int j = 0; j < 3; ++j) {
            const uint64_t blocs = uint64_t(dims->lignes[j]) * (dims->colonnes[j] / 32);
            tc = std::max<uint32_t>(tc, uint32_t(((blocs * 16 + 127) / 128 + n_codes - 1) / n_codes));
        }
        constexpr uint32_t tuiles_bloc = trc::PF_FILS_RAPIDE / 32 * trc::PF_PAIRES_RAPIDE;
        TRC_LANCER(prefill_emplacements_delta_interne, dim3((tc + tuiles_bloc - 1) / tuiles_bloc, 3, experts),
                   dim3(trc::PF_FILS_RAPIDE), f, pp, l, ctl);
    } else if (pp.emplacements != 0) {
        // long tiles: every chosen expert decoded once into its slot (scales, then codes), grids of
        // tile pairs over the largest of the three matrices (the bodies loop over the tiles)
        uint32_t td = 1, tc = 1;
        for (int j = 0; j < 3; ++j) {
            const uint64_t blocs = uint64_t(dims->lignes[j]) * (dims->colonnes[j] / 32);
            td = std::max<uint32_t>(td, uint32_t(((blocs + 127) / 128 + n_delta - 1) / n_delta));
            tc = std::max<uint32_t>(tc, uint32_t(((blocs * 16 + 127) / 128 + n_codes - 1) / n_codes));
        }
        constexpr uint32_t tuiles_d = trc::FILS_ECHELLES / 32, tuiles_c = trc::PF_FILS_CODES_SLOT / 32;
        TRC_LANCER(prefill_emplacements_echelles, dim3((td + tuiles_d - 1) / tuiles_d, 3, experts),
                   dim3(trc::FILS_ECHELLES), f, pp, l, ctl);
        TRC_LANCER(prefill_emplacements_codes, dim3((tc + tuiles_c - 1) / tuiles_c, 3, experts),
                   dim3(trc::PF_FILS_CODES_SLOT), f, pp, l, ctl);
    } else {
        r = trc::lancer_echelles_prefill(pm, Rm, C, n_delta, l, ctl, f);
        if (r != TRC_OK) return r;
    }
    if (pp.emplacements != 0)
        TRC_LANCER(prefill_bande_gu_emplacement, dim3((R + trc::PFE_RB - 1) / trc::PFE_RB, 2 * experts),
                   dim3(trc::PFE_FILS), f, pp, ctl);
    else
        TRC_LANCER(prefill_mfma_gu, dim3((R + pp.rb[0] - 1) / pp.rb[0], 2 * experts), dim3(trc::PF_FILS), f, pp, l, ctl);
    TRC_LANCER(prefill_swiglu_quant, dim3(T * k), dim3(trc::PF_Q_FILS), f, pp);
    if (pp.emplacements != 0)
        TRC_LANCER(prefill_mfma_bas_emplacement, dim3((D + pp.rb[2] - 1) / pp.rb[2], experts), dim3(trc::PF_FILS), f,
                   pp, l, ctl);
    else
        TRC_LANCER(prefill_mfma_bas, dim3((D + pp.rb[2] - 1) / pp.rb[2], experts), dim3(trc::PF_FILS), f, pp, l, ctl);
    const uint32_t fils_comb = pp.quatre ? D / 4u : D;  // threads per position
    TRC_LANCER(prefill_combiner, dim3((fils_comb + 255) / 256, T), dim3(256), f, pp);
    return TRC_OK;
}
