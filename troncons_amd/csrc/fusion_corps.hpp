// fusion_corps.hpp — bodies of the fused-path kernels (gfx950): the DELTA pass that rebuilds the
// E8M0 scales (and each block's CODES_CTX context), and the CODES_CTX pass that decodes the code
// bytes into registers and multiplies them against x on the fly.
//
// Mapping: one wavefront = two rANS tiles (lanes 0-31, 32-63), each tile's words staged in an LDS
// ring (anneau.hpp). In a macro-step, lane v of a tile produces the 4 code bytes 4(v%4) ..
// 4(v%4)+3 of block 8m + v/4, i.e. the weights of columns 32b + 4(v%4) + k (low nibbles) and
// 32b + 16 + 4(v%4) + k (high nibbles): two float4 of x. Each lane accumulates its block
// contributions per row; rows are closed by a 32-lane reduction when the tile's first block enters
// a new row (a row has >= 8 blocks, so one macro-step touches at most two rows). Every (row, tile)
// partial is written exactly once and summed in tile order by the finisher: results are
// deterministic, without floating-point atomics.
#pragma once

#include <type_traits>

#include "anneau.hpp"
#include "commun.hpp"
#include "entiers.hpp"

namespace trc {

// One matrix j of a level-0 part, its four streams located and their headers checked: what every
// fused kernel needs of a part. A mounted layer keeps one per (expert, matrix) in device memory
// (trc_monter_couche), so that per-token kernels read 128 bytes instead of walking the part; the
// single-part entry points build it in each block (analyser_matrice).
struct MatricePartie {
    DescFlux delta, codes, med, biais;
    uint32_t dP, dN, dT, dW;  // DELTA stream header
    uint32_t cP, cN, cT, cW;  // CODES_CTX stream header
    uint32_t bon;             // 1: every check of the reference reader passed
    uint32_t div_m, div_s;    // Diviseur of the blocks per row (multiplier; shifts s1 | s2 << 8)
    uint32_t reserve[5];
};
static_assert(sizeof(MatricePartie) == 128, "MatricePartie");

// Whole wavefront, uniform arguments: the checks of the reference's device reader
// (commun.cuh:101-165, decodeur.cuh:44-70) for matrix j (R x C) of the part.
__device__ inline MatricePartie analyser_matrice(const uint8_t* partie, uint32_t j, uint32_t R, uint32_t C) {
    MatricePartie m;
    m.bon = 0;
    m.dP = m.dN = m.dT = m.dW = m.cP = m.cN = m.cT = m.cW = 0;
    m.div_m = m.div_s = 0;
    const uint32_t B = C / 32u;
    DescFlux f[4];
    const uint8_t sortes[4] = {SORTE_DELTA, SORTE_CODES_CTX, SORTE_MEDIANES, SORTE_BIAIS};
    if (R == 0 || C % 32u != 0 || B == 0 || !trouver_flux_n(partie, sortes, 4, j, f)) return m;
    m.delta = f[0];
    m.codes = f[1];
    m.med = f[2];
    m.biais = f[3];
    EnteteRans hd, hc;
    const bool bon = lire_entete(f[0], R * B, hd) && lire_entete(f[1], R * B * 16u, hc) && f[2].produits == R &&
                     f[2].longueur >= R && f[3].produits == 4u * R && f[3].longueur >= 4u * R;
    if (!bon) return m;
    m.dP = hd.P;
    m.dN = hd.N;
    m.dT = hd.T;
    m.dW = hd.W;
    m.cP = hc.P;
    m.cN = hc.N;
    m.cT = hc.T;
    m.cW = hc.W;
    const Diviseur dv = Diviseur::de(B);  // once per matrix, where the record is made
    m.div_m = dv.m;
    m.div_s = dv.s1 | (dv.s2 << 8);
    m.bon = 1;
    return m;
}

// Entry of one block (u32), written by the DELTA pass and read by the CODES pass:
//   bits 7-13   column block b (x byte offset b * 128 in the LDS copy of x; 127 = the zero slot),
//   bits 15-16  context kappa (LUT byte offset kappa * 32 KiB),
//   bits 17-24  e - 128 as a signed byte (the block's scale is 2^(e-128)),
//   bit 31      the block starts a row (b == 0).
// Rows wider than 127 blocks keep b & 127 there (the device-memory-x variant recomputes b).
constexpr uint32_t ENT_X = 0x3F80u;
constexpr uint32_t ENT_CTX = 0x18000u;
constexpr uint32_t ENT_EXP = 17u;
constexpr uint32_t ENT_LIGNE = 0x80000000u;
constexpr uint32_t COLONNE_NULLE = 127u;
__host__ __device__ __forceinline__ uint32_t entree_bloc(uint32_t e, uint32_t ctx, uint32_t b, bool debut_ligne) {
    return ((b & 127u) << 7) | (ctx << 15) | (((e - 128u) & 0xFFu) << ENT_EXP) | (debut_ligne ? ENT_LIGNE : 0u);
}
// Stream padding past the last block: zero x slot, scale 1, context 0.
constexpr uint32_t ENTREE_BOURRAGE = COLONNE_NULLE << 7;

// One job of the fused path: matrix j of a level-0 part, against x (64 bytes).
struct Tache {
    uint64_t partie;    // level-0 part (read when `matrice` is 0)
    uint64_t matrice;   // MatricePartie of a mounted layer, or 0
    uint64_t x;         // f32[colonnes], 16-byte aligned
    uint64_t ech;       // u32[lignes * colonnes/32 + ECH_MARGE] block entries (workspace)
    uint64_t partiels;  // f32[lignes * kmax] partial sums (workspace)
    uint32_t j;         // matrix index in the part
    uint32_t kmax;      // partial slots per row
    uint32_t lignes, colonnes;
    uint32_t reserve[2];
};
static_assert(sizeof(Tache) == 64, "Tache");

// Stores a MatricePartie field by field (a struct copy would take the address of a value that
// lives in registers and move it to scratch).
__device__ __forceinline__ u32x4 quad_flux(const DescFlux& f) {
    const uint64_t a = reinterpret_cast<uintptr_t>(f.p);
    return u32x4{uint32_t(a), uint32_t(a >> 32), f.longueur, f.produits};
}
__device__ __forceinline__ void ecrire_matrice(void* dst, const MatricePartie& m) {
    __attribute__((address_space(1))) u32x4* d = (__attribute__((address_space(1))) u32x4*)(dst);
    d[0] = quad_flux(m.delta);
    d[1] = quad_flux(m.codes);
    d[2] = quad_flux(m.med);
    d[3] = quad_flux(m.biais);
    d[4] = u32x4{m.dP, m.dN, m.dT, m.dW};
    d[5] = u32x4{m.cP, m.cN, m.cT, m.cW};
    d[6] = u32x4{m.bon, m.div_m, m.div_s, 0u};
    d[7] = u32x4{0u, 0u, 0u, 0u};
}

// The job's matrix: from the mounted layer (one 128-byte read) or parsed from the part.
__device__ __forceinline__ MatricePartie obtenir_matrice(const Tache& tc) {
    if (tc.matrice != 0) return *reinterpret_cast<const MatricePartie*>(tc.matrice);
    return analyser_matrice(reinterpret_cast<const uint8_t*>(tc.partie), tc.j, tc.lignes, tc.colonnes);
}

// The same, a resolved record read with scalar loads (constant address space): it lands in SGPRs
// and is waited for on the scalar counter, so vector loads in flight are not drained for it. Only
// for records that nothing writes while the kernel runs (the layer's directory, or the selected
// experts' records written by an earlier launch).
__device__ __forceinline__ MatricePartie lire_matrice_constante(uint64_t adresse) {
#if defined(__HIP_DEVICE_COMPILE__)
    typedef const __attribute__((address_space(4))) MatricePartie* MatriceConstante;
    const MatricePartie m = *reinterpret_cast<MatriceConstante>(adresse);
    return m;
#else
    return *reinterpret_cast<const MatricePartie*>(adresse);  // host pass of a device function: never run
#endif
}
// The same, its seven 16-byte words (the eighth is reserve) read with scalar loads that are all
// issued before any is used: the empty asm takes every word (and `extra`, values the caller read
// just before, such as other records' fields), so one wait covers them all. Without it the
// compiler moves each field's load down to its first use, one round trip after another.
__device__ __forceinline__ MatricePartie lire_matrice_groupee(uint64_t adresse, u32x4& extra) {
    struct Mots {
        u32x4 w[8];
    } m;
#if defined(__HIP_DEVICE_COMPILE__)
    typedef const __attribute__((address_space(4))) u32x4* MotsConstants;
    const MotsConstants q = reinterpret_cast<MotsConstants>(adresse);
#pragma unroll
    for (uint32_t k = 0; k < 7u; ++k) m.w[k] = q[k];
    asm volatile("" : "+s"(m.w[0]), "+s"(m.w[1]), "+s"(m.w[2]), "+s"(m.w[3]), "+s"(m.w[4]), "+s"(m.w[5]),
                 "+s"(m.w[6]), "+s"(extra));
#else
    const u32x4* q = reinterpret_cast<const u32x4*>(adresse);  // host pass of a device function: never run
    for (uint32_t k = 0; k < 7u; ++k) m.w[k] = q[k];
#endif
    m.w[7] = u32x4{0u, 0u, 0u, 0u};
    static_assert(sizeof(Mots) == sizeof(MatricePartie), "a record is 8 words");
    return __builtin_bit_cast(MatricePartie, m);
}

// One u32 of such a record, by a scalar load.
__device__ __forceinline__ uint32_t lire_u32_constante(uint64_t adresse) {
#if defined(__HIP_DEVICE_COMPILE__)
    return *reinterpret_cast<const __attribute__((address_space(4))) uint32_t*>(adresse);
#else
    return *reinterpret_cast<const uint32_t*>(adresse);  // host pass of a device function: never run
#endif
}
__device__ __forceinline__ MatricePartie obtenir_matrice_scalaire(const Tache& tc) {
    if (tc.matrice != 0) return lire_matrice_constante(tc.matrice);
    return analyser_matrice(reinterpret_cast<const uint8_t*>(tc.partie), tc.j, tc.lignes, tc.colonnes);
}

// A MoE layer's jobs, derived on the device from the router's top-k: selected expert i (index
// indices[i] < E, else its jobs get no matrix and count as format errors) has matrices j = 0, 1, 2
// (gate, up, down), each with its own workspace piece (i*3 + j) * pas; gate/up read x, down reads
// expert i's SwiGLU row (act, finished once per expert between the gate/up and down passes).
struct ParamsMoe {
    uint64_t repertoire;  // MatricePartie[E][3] of the mounted layer
    uint64_t resolus;     // MatricePartie[k][3] of the selected experts, copied by the DELTA pass
    uint64_t logits;      // f32[E] router logits (the DELTA pass runs the top-k on them)
    uint64_t indices;     // u32[k] top-k indices, written by the DELTA pass
    uint64_t poids;       // f32[k] softmax weights, written by the DELTA pass
    uint64_t x;           // f32[C]
    uint64_t residu;      // f32[D] the combine adds into
    uint64_t ech;         // scale entries of piece 0
    uint64_t partiels;    // partial sums of piece 0
    uint64_t pas;         // workspace bytes per piece
    uint64_t compte;      // (prefill) u32[E] positions that chose expert e; experts with 0 are skipped
    uint64_t act;         // f32[k][colonnes[2]] the experts' SwiGLU rows, the down jobs' x (0: built by the down pass)
    uint64_t biais;       // f32[k][3][max(lignes)] the selected matrices' biases, copied by their CODES passes
                          // (OPT_BIAIS), so that later launches read them without the records
    uint32_t lignes[3], colonnes[3], kmax[3];
    uint32_t k, E;
};

enum ModeTaches : uint32_t {
    TACHES_LOCALES = 0,  // up to 3 jobs passed by value (one matrix, one expert)
    TACHES_MOE_DELTA = 1,  // job y = (expert y/3, matrix y%3)
    TACHES_MOE_GU = 2,     // job y = (expert y/2, matrix y%2)
    TACHES_MOE_BAS = 3,    // job y = (expert y, matrix 2)
    TACHES_PREFILL_DELTA = 4,  // job y = (expert y/3, matrix y%3), workspace piece y, if chosen
};


// Job (expert i = expert e of the layer, matrix j) of a MoE layer.
__device__ __forceinline__ Tache tache_moe_e(const ParamsMoe& moe, uint32_t i, uint32_t j, uint32_t e) {
    Tache t;
    t.partie = 0;
    t.matrice = e < moe.E ? moe.repertoire + uint64_t(e * 3u + j) * sizeof(MatricePartie) : 0ull;
    t.j = j;
    t.kmax = choisir(moe.kmax, j);
    t.lignes = choisir(moe.lignes, j);
    t.colonnes = choisir(moe.colonnes, j);
    t.ech = moe.ech + uint64_t(i * 3u + j) * moe.pas;
    t.partiels = moe.partiels + uint64_t(i * 3u + j) * moe.pas;
    t.x = j < 2u ? moe.x : (moe.act != 0 ? moe.act + 4ull * i * moe.colonnes[2] : 0ull);
    t.reserve[0] = t.reserve[1] = 0;
    return t;
}

// Job (expert i, matrix j) of the later passes: the matrix is the one the DELTA pass resolved and
// copied into the workspace, so no pass after it reads the top-k or the directory again.
__device__ __forceinline__ Tache tache_moe(const ParamsMoe& moe, uint32_t i, uint32_t j) {
    Tache t = tache_moe_e(moe, i, j, 0u);
    t.matrice = moe.resolus + uint64_t(i * 3u + j) * sizeof(MatricePartie);
    return t;
}

// The jobs of a launch; job of block (x, y) = y.
struct Taches {
    Tache locales[3];
    ParamsMoe moe;
    uint32_t mode;
    uint32_t options;
    __device__ __forceinline__ Tache operator[](uint32_t y) const {
        if (mode == TACHES_LOCALES) return locales[y];
        uint32_t i, j;
        if (mode == TACHES_MOE_DELTA) {
            i = y / 3u;
            j = y - 3u * i;
        } else if (mode == TACHES_MOE_GU) {
            i = y >> 1;
            j = y & 1u;
        } else {
            i = y;
            j = 2u;
        }
        return tache_moe(moe, i, j);
    }
};

#ifndef TRC_FILS_ECHELLES
#define TRC_FILS_ECHELLES 1024
#endif
constexpr uint32_t FILS_ECHELLES_FUSION = TRC_FILS_ECHELLES;  // default 16 wavefronts, 32 DELTA tiles
static_assert(FILS_ECHELLES_FUSION % 64 == 0 && FILS_ECHELLES_FUSION <= 1024, "whole wavefronts, one block");
// LUT loads in flight per thread when a DELTA block stages its 4096-entry table (one 16-byte load
// per thread at 1024 threads)
constexpr uint32_t LOT_LUT_ECHELLES = (1024u + FILS_ECHELLES_FUSION - 1u) / FILS_ECHELLES_FUSION;
constexpr uint32_t FILS_GEMV_MAX = 1024;        // up to 16 wavefronts, 32 CODES_CTX tiles
constexpr uint32_t ENT_PAR_TUILE = 128;         // block entries staged per tile (16 macro-steps)
constexpr uint32_t ECH_MARGE = 256;             // entries past the last block that staging may read
constexpr uint32_t X_LDS_MAX = 4064;            // columns of x the CODES pass keeps in LDS (127 blocks)

// LDS of the CODES pass: one array aligned on 16 KiB, so that every region base keeps the alignment
// the address arithmetic relies on (x: 16 KiB, rings: 1 KiB).
constexpr uint32_t LDS_LUT = 0;                                  // 3 contexts x 4096 x 8 B
constexpr uint32_t LDS_X = 3u * 4096u * 8u;                      // x (f32) + the zero slot: 16 KiB
constexpr uint32_t LDS_ANNEAUX = LDS_X + 16384u;                 // 32 rings x 1 KiB
constexpr uint32_t LDS_ENT = LDS_ANNEAUX + 32u * OCTETS_ANNEAU;  // 32 tiles x 128 entries x 4 B
constexpr uint32_t LDS_GEMV = LDS_ENT + 32u * ENT_PAR_TUILE * 4u;
static_assert(LDS_GEMV == 160u * 1024u, "the CODES pass uses all 160 KiB of a CU's LDS");
constexpr uint32_t MED_LDS_MAX = 8192;          // rows whose medians the DELTA pass keeps in LDS

// A job read by every lane (same address) made wave-uniform, so that the part reader and all the
// job's scalars live in scalar registers. (The builtin returns int; elargir_u64 widens each half
// through uint32_t, so that an address whose low word has bit 31 set is not sign-extended.)
__device__ __forceinline__ uint32_t uniforme32(uint32_t v) { return uint32_t(__builtin_amdgcn_readfirstlane(v)); }
// Workgroup barrier that orders LDS accesses only. __syncthreads() fences every address space, so
// each wave first waits for all of its outstanding device-memory loads; this one leaves loads that
// are meant to stay in flight across the barrier (read-ahead of the first tiles) in flight.
__device__ __forceinline__ void barriere_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
__device__ __forceinline__ uint64_t uniforme64(uint64_t v) {
    return elargir_u64(__builtin_amdgcn_readfirstlane(uint32_t(v)), __builtin_amdgcn_readfirstlane(uint32_t(v >> 32)));
}
__device__ __forceinline__ Tache uniforme(const Tache& t) {
    Tache u;
    u.partie = uniforme64(t.partie);
    u.matrice = uniforme64(t.matrice);
    u.x = uniforme64(t.x);
    u.ech = uniforme64(t.ech);
    u.partiels = uniforme64(t.partiels);
    u.j = uniforme32(t.j);
    u.kmax = uniforme32(t.kmax);
    u.lignes = uniforme32(t.lignes);
    u.colonnes = uniforme32(t.colonnes);
    return u;
}

__device__ __forceinline__ uint32_t premiere_tuile(uint32_t ligne, uint32_t B, uint32_t blocs_par_tuile) {
    return (ligne * B) / blocs_par_tuile;
}

template <typename T>
__device__ __forceinline__ void ecrire_global(void* p, T v) {
    *(__attribute__((address_space(1))) T*)(p) = v;
}
// The same with the nontemporal hint (data read back by another launch: no reuse in the L2).
template <typename T>
__device__ __forceinline__ void ecrire_global_nt(void* p, T v) {
    __builtin_nontemporal_store(v, (__attribute__((address_space(1))) T*)(p));
}

// Context class of a block from its DELTA symbol (decodeur.cuh:185-192, rans.rs:481-486).
__device__ __forceinline__ uint32_t classe_delta(uint32_t d) { return d < 128u ? 0u : (d == 128u ? 1u : 2u); }

// ----------------------------------------------------------------------------- DELTA pass
struct PrepEchelles {
    DescFlux fd, fm;
    EnteteRans h;
    bool bon;
};

// A tile's head: its lanes' initial states, its first word, and the word its decode must end on
// (the next tile's first, or W). Read one tile ahead, so that no decode waits for these loads.
// LDS addresses (32-bit) of an LDS array.
typedef __attribute__((address_space(3))) uint8_t lds_u8;
__device__ __forceinline__ uint32_t adresse_lds(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((const lds_u8*)(p)));  // address-space cast
}
template <typename T>
__device__ __forceinline__ T lire_lds(uint32_t a) {
    return *reinterpret_cast<const __attribute__((address_space(3))) T*>(uintptr_t(a));
}
template <typename T>
__device__ __forceinline__ void ecrire_lds(uint32_t a, T v) {
    *reinterpret_cast<__attribute__((address_space(3))) T*>(uintptr_t(a)) = v;
}

struct TeteTuile {
    uint32_t x, debut, attendu;
};

__device__ __forceinline__ TeteTuile lire_tete(const EnteteRans& h, uint32_t t, uint32_t v) {
    TeteTuile r{L, 0u, 0u};
    if (t < h.T) {
        r.x = h.etats[t * VOIES + v];
        r.debut = h.debut[t];
        r.attendu = (t + 1u < h.T) ? h.debut[t + 1u] : h.W;
    }
    return r;
}

// The same with its loads unconditional (tile index clamped to the last tile, h.T >= 1), so that no
// branch surrounds them: a tile past the stream gets the last tile's head, which its half never
// decodes nor checks.
__device__ __forceinline__ TeteTuile lire_tete_borne(const EnteteRans& h, uint32_t t, uint32_t v) {
    const uint32_t tt = min(t, h.T - 1u);
    const gptr<uint32_t> debut = glob<uint32_t>(h.debut);
    const uint32_t apres = debut[min(tt + 1u, h.T - 1u)];
    TeteTuile r;
    r.x = glob<uint32_t>(h.etats)[tt * VOIES + v];
    r.debut = debut[tt];
    r.attendu = tt + 1u < h.T ? apres : h.W;
    return r;
}

// The head of the first tile of the calling lane's half-wavefront (the tile loops below start at
// tile 2 * (global wavefront index), the upper half one further).
__device__ __forceinline__ TeteTuile premiere_tete(const EnteteRans& h) {
    const uint32_t vague = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    return lire_tete(h, 2u * vague + (__lane_id() >= 32u ? 1u : 0u), __lane_id() & 31u);
}

__device__ __forceinline__ PrepEchelles preparer_echelles(const Tache& tc, const MatricePartie& m) {
    PrepEchelles p;
    p.bon = m.bon != 0 && tc.colonnes % 32u == 0 && tc.colonnes >= 32u && tc.lignes > 0;
    p.fd = m.delta;
    p.fm = m.med;
    p.h = entete_de(m.delta, m.dP, m.dN, m.dT, m.dW);
    return p;
}

// The DELTA pass gives each half-wavefront a run of consecutive tiles, [t_deb, t_fin): the runs of
// the grid's half-wavefronts split the stream's T tiles evenly. A run's tiles are stored one after
// the other, so one word ring carries the whole run and is opened once.
constexpr uint32_t ECH_KMAX = 4;  // tiles of a run whose initial states are held in registers at once

__device__ __forceinline__ void course_echelles(uint32_t T, uint32_t& t_deb, uint32_t& t_fin) {
    const uint32_t D = gridDim.x * (blockDim.x >> 5), d = blockIdx.x * (blockDim.x >> 5) + (threadIdx.x >> 5);
    t_deb = uint32_t(uint64_t(T) * d / D);
    t_fin = uint32_t(uint64_t(T) * (d + 1u) / D);
}

// The run's word origin (debut[t_deb]) in `debut` and the word where it must end (debut[t_fin], or W
// at the stream's end) in `attendu`; loads clamped, so that no branch surrounds them.
__device__ __forceinline__ TeteTuile tete_course(const EnteteRans& h) {
    uint32_t t_deb, t_fin;
    course_echelles(h.T, t_deb, t_fin);
    const gptr<uint32_t> debut = glob<uint32_t>(h.debut);
    TeteTuile r;
    r.x = L;
    r.debut = debut[min(t_deb, h.T - 1u)];
    const uint32_t fin = debut[min(t_fin, h.T - 1u)];
    r.attendu = t_fin < h.T ? fin : h.W;
    return r;
}

// DELTA tiles -> one entry per block (entree_bloc) with e = (med[row] + delta - 128) mod 256 and
// kappa = the class of delta; blocks past the matrix (stream padding) get the padding entry. Each
// tile starts from its own initial states and must end in state L, its word pointer on the next
// tile's first word (or W after the last tile), as the reference checks every tile
// (commun.cuh:240-246, rans.rs:442-448): a run's ring carries the words across its tiles, so a tile
// start inside the run is checked where the previous tile ends. The medians are read from LDS
// (MED_LDS = true: med_lds holds them) or from the stream. A lane's 4 blocks of a macro-step lie in
// at most two rows when B >= 4; narrower rows take a loop. `tete0`: tete_course(p.h), read by the
// caller before its barrier.
template <bool MED_LDS>
__device__ __forceinline__ void corps_echelles_fusion(const Tache& tc, const PrepEchelles& p, const uint2* lut,
                                                      const uint8_t* med_lds, uint8_t* anneaux,
                                                      uint32_t* __restrict__ controle, const TeteTuile& tete0) {
    const EnteteRans& h = p.h;
    const uint32_t R = tc.lignes, B = tc.colonnes / 32u, nblocs = R * B;
    const uint32_t a_med = adresse_lds(med_lds);
    const gptr<uint8_t> med_g = glob<uint8_t>(p.fm.p);
    auto mediane = [&](uint32_t r) -> uint32_t {  // r < R
        return MED_LDS ? uint32_t(lire_lds<uint8_t>(a_med + r)) : uint32_t(med_g[r]);
    };
    const uint32_t q128 = 128u / B, r128 = 128u - q128 * B;  // a macro-step's 128 blocks per lane group
    uint32_t* ech = reinterpret_cast<uint32_t*>(tc.ech);
    const uint32_t lane = __lane_id();
    const uint32_t v = lane & 31u;
    const bool haut = lane >= 32u;
    const uint32_t decal = haut ? 32u : 0u, masque_inf = (1u << v) - 1u;
    const uint32_t lds = (threadIdx.x >> 5) * OCTETS_ANNEAU;
    const uint32_t N = h.N, nmacro = h.P / 128u;
    uint32_t t_deb, t_fin;
    course_echelles(h.T, t_deb, t_fin);
    const uint32_t nt = t_fin - t_deb;
    // the wave's two runs, for wave-uniform loop bounds
    const uint32_t nt_lo = uint32_t(__builtin_amdgcn_readlane(int(nt), 0));
    const uint32_t nt_hi = uint32_t(__builtin_amdgcn_readlane(int(nt), 32));
    const uint32_t td_lo = uint32_t(__builtin_amdgcn_readlane(int(t_deb), 0));
    const uint32_t td_hi = uint32_t(__builtin_amdgcn_readlane(int(t_deb), 32));
    const uint32_t nt_max = max(nt_lo, nt_hi);
    Anneau a = ouvrir_anneau(h, p.fd, tete0.debut, lds, anneaux, v, nt > 0u);
    const uint32_t o0 = a.o2;
    uint32_t x = L;
    uint32_t hors_l = 0, pointeur = 0;
    uint32_t b0 = 4u * (t_deb * N * VOIES + v);
    uint32_t ligne = b0 / B, reste = b0 - ligne * B;
    auto macro = [&](auto tous, bool actif_t) {
        constexpr bool TOUS = decltype(tous)::value;
        const bool actif = TOUS || actif_t;
        uint32_t mot = 0;
#pragma unroll
        for (uint32_t k = 0; k < 4; ++k)
            mot |= (pas_anneau<TOUS>(x, a, lut, anneaux, decal, masque_inf, actif) >> 24) << (8u * k);
        avancer_anneau(a, anneaux, v, actif);
        if (actif) {
            u32x4 sortie;
            if (B >= 4u) {  // uniform
                const uint32_t m0 = ligne < R ? mediane(ligne) : 0u;
                const uint32_t m1 = ligne + 1u < R ? mediane(ligne + 1u) : 0u;
#pragma unroll
                for (uint32_t k = 0; k < 4; ++k) {
                    const bool suivante = reste + k >= B;
                    const uint32_t qk = reste + k - (suivante ? B : 0u);
                    const uint32_t d = (mot >> (8u * k)) & 255u;
                    const uint32_t mk = suivante ? m1 : m0;
                    sortie[k] = b0 + k < nblocs
                                    ? entree_bloc((mk + d - 128u) & 255u, classe_delta(d), qk, qk == 0u)
                                    : ENTREE_BOURRAGE;
                }
            } else {
#pragma unroll
                for (uint32_t k = 0; k < 4; ++k) {
                    uint32_t rk = ligne, qk = reste + k;
                    while (qk >= B) {
                        qk -= B;
                        ++rk;
                    }
                    const uint32_t d = (mot >> (8u * k)) & 255u;
                    const uint32_t mk = rk < R ? mediane(rk) : 0u;
                    sortie[k] = b0 + k < nblocs
                                    ? entree_bloc((mk + d - 128u) & 255u, classe_delta(d), qk, qk == 0u)
                                    : ENTREE_BOURRAGE;
                }
            }
            ecrire_global<u32x4>(ech + b0, sortie);  // the workspace covers the stream's padding
            b0 += 4u * VOIES;
            ligne += q128;
            reste += r128;
            if (reste >= B) {
                reste -= B;
                ++ligne;
            }
        }
    };
    const gptr<uint32_t> etats = glob<uint32_t>(h.etats);
    const gptr<uint32_t> debuts = glob<uint32_t>(h.debut);
    // the initial states of ECH_KMAX tiles at a time, with the first word of the tile after each
    // (where each must end); the next group's are requested while the current group decodes
    uint32_t suiv[ECH_KMAX], suiv_fin[ECH_KMAX];
#pragma unroll
    for (uint32_t kk = 0; kk < ECH_KMAX; ++kk) {
        suiv[kk] = etats[min(t_deb + kk, h.T - 1u) * VOIES + v];
        suiv_fin[kk] = debuts[min(t_deb + kk + 1u, h.T - 1u)];
    }
    for (uint32_t k0 = 0; k0 < nt_max; k0 += ECH_KMAX) {  // wave-uniform
        uint32_t etat[ECH_KMAX], fin_mots[ECH_KMAX];
#pragma unroll
        for (uint32_t kk = 0; kk < ECH_KMAX; ++kk) {
            etat[kk] = suiv[kk];
            fin_mots[kk] = suiv_fin[kk];
        }
        if (k0 + ECH_KMAX < nt_max) {  // wave-uniform
#pragma unroll
            for (uint32_t kk = 0; kk < ECH_KMAX; ++kk) {
                suiv[kk] = etats[min(t_deb + k0 + ECH_KMAX + kk, h.T - 1u) * VOIES + v];
                suiv_fin[kk] = debuts[min(t_deb + k0 + ECH_KMAX + kk + 1u, h.T - 1u)];
            }
        }
#pragma unroll
        for (uint32_t kk = 0; kk < ECH_KMAX; ++kk) {
            const uint32_t k = k0 + kk;
            if (k >= nt_max) break;  // wave-uniform
            // macro-steps of the two halves' k-th tiles (0 past a run's end), wave-uniform
            const uint32_t nb_lo = k < nt_lo ? min(N, nmacro - (td_lo + k) * N) : 0u;
            const uint32_t nb_hi = k < nt_hi ? min(N, nmacro - (td_hi + k) * N) : 0u;
            const uint32_t nb = haut ? nb_hi : nb_lo;
            const bool tuile = k < nt;
            if (tuile) x = etat[kk];
            const uint32_t nb_min = min(nb_lo, nb_hi), nb_max = max(nb_lo, nb_hi);
            uint32_t m = 0;
            for (; m < nb_min; ++m) macro(std::true_type{}, true);
            for (; m < nb_max; ++m) macro(std::false_type{}, m < nb);
            if (tuile) {
                hors_l += (x != L) ? 1u : 0u;
                const uint32_t attendu = t_deb + k + 1u < h.T ? fin_mots[kk] : h.W;
                pointeur += (v == 0 && tete0.debut + (a.o2 - o0) / 2u != attendu) ? 1u : 0u;
            }
        }
    }
    verser_controle(controle, hors_l, pointeur);
}

// ------------------------------------------------------------------------- CODES_CTX pass
struct PrepGemv {
    DescFlux fc;
    EnteteRans h;
    bool bon;
};

__device__ __forceinline__ PrepGemv preparer_gemv(const Tache& tc, const MatricePartie& m) {
    const uint32_t B = tc.colonnes / 32u;
    PrepGemv p;
    p.bon = m.bon != 0 && tc.colonnes % 32u == 0 && B >= 8u && tc.lignes > 0 &&
            (B - 1u) / (8u * m.cN) + 2u <= tc.kmax;  // enough partial slots per row
    p.fc = m.codes;
    p.h = entete_de(m.codes, m.cP, m.cN, m.cT, m.cW);
    return p;
}

// Row bookkeeping shared by both CODES bodies: the (row, tile) partial slot of row r for tile t.
__device__ __forceinline__ void ecrire_partiel(float* partiels, uint32_t kmax, uint32_t r, uint32_t t, uint32_t B,
                                               uint32_t bpt, float s) {
    ecrire_global<float>(partiels + r * kmax + (t - premiere_tuile(r, B, bpt)), s);
}

// CODES_CTX tiles -> partial sums of W x with x read from device memory (rows of any width; the
// column of each block is tracked per lane). ent_lds: ENT_PAR_TUILE entries per half-wavefront.
__device__ __forceinline__ void corps_gemv_xg(const Tache& tc, const PrepGemv& p, const uint2* lut, uint8_t* anneaux,
                                              uint32_t* ent_lds, uint32_t* __restrict__ controle) {
    const EnteteRans& h = p.h;
    const uint32_t R = tc.lignes, B = tc.colonnes / 32u, nblocs = R * B;
    const gptr<u32x4> ent16 = glob<u32x4>(reinterpret_cast<const void*>(tc.ech));
    const gptr<f32x4> xg = glob<f32x4>(reinterpret_cast<const void*>(tc.x));
    float* __restrict__ partiels = reinterpret_cast<float*>(tc.partiels);
    const uint32_t kmax = tc.kmax;
    const uint32_t bpt = 8u * h.N;  // blocks per tile

    const uint32_t lane = __lane_id();
    const uint32_t v = lane & 31u;
    const bool haut = lane >= 32u;
    const uint32_t decal = haut ? 32u : 0u, masque_inf = (1u << v) - 1u;
    const uint32_t q = v >> 2, q4 = v & 3u;
    const uint32_t vagues_bloc = blockDim.x >> 6;
    // wave-uniform (scalar registers): the tile loop and its macro-step counts run on SALU
    const uint32_t vague = uniforme32(blockIdx.x * vagues_bloc + (threadIdx.x >> 6));
    const uint32_t n_vagues = gridDim.x * vagues_bloc;
    const uint32_t demi = (threadIdx.x >> 5) & (2u * vagues_bloc - 1u);
    const uint32_t lds = demi * OCTETS_ANNEAU;
    uint32_t* mes_ent = ent_lds + demi * ENT_PAR_TUILE;
    const uint32_t nmacro = h.P / 128u;
    uint32_t hors_l = 0, pointeur = 0;
    for (uint32_t t0 = 2u * vague; t0 < h.T; t0 += 2u * n_vagues) {
        const uint32_t t = t0 + (haut ? 1u : 0u);
        const bool tuile = t < h.T;
        const uint32_t nb_a = min(h.N, nmacro - t0 * h.N);
        const uint32_t nb_b = (t0 + 1u < h.T) ? min(h.N, nmacro - (t0 + 1u) * h.N) : 0u;
        const uint32_t nb = haut ? nb_b : nb_a;
        const uint32_t m0 = (tuile ? t : t0) * h.N;
        // entries of macro-steps m .. m+15 of the tile: blocks 8(m0+m) .. +127, 4 per lane (the
        // workspace holds ECH_MARGE entries past the last block, so the load stays inside it)
        auto stager = [&](uint32_t m) { *reinterpret_cast<u32x4*>(mes_ent + 4u * v) = ent16[2u * (m0 + m) + v]; };
        uint32_t x = tuile ? h.etats[t * VOIES + v] : L;
        const uint32_t debut = tuile ? h.debut[t] : 0u;
        if (tuile) stager(0);
        Anneau a = ouvrir_anneau(h, p.fc, debut, lds, anneaux, v, tuile);
        const uint32_t o0 = a.o2;
        uint32_t bloc = m0 * 8u + q;
        uint32_t ligne = bloc / B, b = bloc - ligne * B;
        uint32_t rho = (m0 * 8u) / B, base_b = m0 * 8u - rho * B;  // row of the tile's first block
        bool valide = tuile && bloc < nblocs;
        uint32_t ent_suiv = tuile ? mes_ent[q] : 0u;
        float acc_a = 0.0f, acc_b = 0.0f;
        auto macro = [&](auto tous, uint32_t m) {
            constexpr bool TOUS = decltype(tous)::value;
            const bool actif = TOUS || m < nb;
            const bool bloc_ok = valide;
            const uint32_t ent = ent_suiv;
            const uint32_t b_cur = b;
            const bool ligne_a = ligne == rho;
            f32x4 xa = {0.f, 0.f, 0.f, 0.f}, xb = xa;
            if (bloc_ok) {
                xa = xg[8u * b_cur + q4];
                xb = xg[8u * b_cur + 4u + q4];
            }
            bloc += 8u;
            b += 8u;
            if (b >= B) {  // B >= 8: at most one row per macro-step
                b -= B;
                ++ligne;
            }
            valide = (m + 1u < nb) && bloc < nblocs;
            if (((m + 1u) & 15u) == 0u && m + 1u < nb) stager(m + 1u);
            ent_suiv = mes_ent[(8u * (m + 1u) + q) & (ENT_PAR_TUILE - 1u)];
            const uint2* lt = lut + (bloc_ok ? ((ent & ENT_CTX) >> 15) * M : 0u);
            const uint32_t e0 = pas_anneau<TOUS>(x, a, lt, anneaux, decal, masque_inf, actif);
            const uint32_t e1 = pas_anneau<TOUS>(x, a, lt, anneaux, decal, masque_inf, actif);
            const uint32_t e2 = pas_anneau<TOUS>(x, a, lt, anneaux, decal, masque_inf, actif);
            const uint32_t e3 = pas_anneau<TOUS>(x, a, lt, anneaux, decal, masque_inf, actif);
            avancer_anneau(a, anneaux, v, actif);
            if (actif && bloc_ok) {
                const f32x2 w0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e0, 2.0f, 3);
                const f32x2 w1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e1, 2.0f, 3);
                const f32x2 w2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e2, 2.0f, 3);
                const f32x2 w3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e3, 2.0f, 3);
                float d = w0.x * xa.x;
                d = fmaf(w0.y, xb.x, d);
                d = fmaf(w1.x, xa.y, d);
                d = fmaf(w1.y, xb.y, d);
                d = fmaf(w2.x, xa.z, d);
                d = fmaf(w2.y, xb.z, d);
                d = fmaf(w3.x, xa.w, d);
                d = fmaf(w3.y, xb.w, d);
                const float c = __builtin_amdgcn_ldexpf(d, int(ent << 7) >> 24);  // d * 2^(e-128), exact
                if (ligne_a)
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
            if (__builtin_amdgcn_ballot_w64(avance) != 0) {
                const float s = somme_demi_f32(acc_a);
                if (avance) {
                    if (v == 0 && rho < R) ecrire_partiel(partiels, kmax, rho, t, B, bpt, s);
                    acc_a = acc_b;
                    acc_b = 0.0f;
                    ++rho;
                }
            }
        };
        const uint32_t nb_min = min(nb_a, nb_b);
        uint32_t m = 0;
        for (; m < nb_min; ++m) macro(std::true_type{}, m);
        for (; m < nb_a; ++m) macro(std::false_type{}, m);
        const float sa = somme_demi_f32(acc_a);
        const float sb = somme_demi_f32(acc_b);
        if (tuile) {
            if (v == 0) {
                const uint32_t fin = min((m0 + nb) * 8u, nblocs);
                const uint32_t derniere = (fin - 1u) / B;
                if (rho <= derniere && rho < R) ecrire_partiel(partiels, kmax, rho, t, B, bpt, sa);
                if (rho + 1u <= derniere && rho + 1u < R) ecrire_partiel(partiels, kmax, rho + 1u, t, B, bpt, sb);
            }
            hors_l += (x != L) ? 1u : 0u;
            const uint32_t attendu = (t + 1 < h.T) ? h.debut[t + 1] : h.W;
            pointeur += (v == 0 && debut + (a.o2 - o0) / 2u != attendu) ? 1u : 0u;
        }
    }
    verser_controle(controle, hors_l, pointeur);
}

// ------------------------------------------------- CODES_CTX pass with x in LDS (the hot path)
//
// Same tiles and mapping; everything a macro-step needs besides the words comes from the block's
// entry: the LUT base (context), the address of the two float4 of x (column), the scale and the
// row start. Each lane keeps one accumulator for the tile's current row; a macro-step in which a
// row starts (at most one per half: a row has >= 8 blocks) takes the slow path that closes the
// row. Stream padding blocks read the zero slot of x, so no per-block validity test is needed.

// A tile's word ring (as Anneau, with absolute LDS addresses; `lds` is 1 KiB aligned). Chunks are
// addressed by 32-bit offsets from the stream's start, which both tiles of a wavefront share.
struct AnneauR {
    const uint8_t* flux;  // start of the stream (its descriptor's p)
    uint32_t g0;      // offset from `flux` of the tile's 16-byte aligned word origin
    uint32_t fin;     // length of the stream: chunk loads never pass it
    uint32_t lds;     // LDS address of the ring
    uint32_t o2;      // byte offset from g0 of the next word (unwrapped)
    uint32_t limite;  // refill when o2 > limite (= charge * 256 - FENETRE)
    uint32_t charge;  // next chunk to request
    u32x2 vol;
    bool en_vol;
};

__device__ __forceinline__ u32x2 lire_morceau_r(const AnneauR& a, uint32_t c, uint32_t v) {
    const uint32_t o = a.g0 + c * OCTETS_MORCEAU + v * 8u;
    u32x2 d = {0u, 0u};
    if (o + 8u <= a.fin) d = *glob<u32x2>(a.flux + o);
    return d;
}

__device__ __forceinline__ AnneauR ouvrir_anneau_r(const EnteteRans& h, const DescFlux& f, uint32_t debut,
                                                   uint32_t lds, uint32_t v, bool tuile) {
    AnneauR a;
    const uint32_t mot0 = uint32_t(reinterpret_cast<const uint8_t*>(h.mots) - f.p) + 2u * debut;
    a.flux = f.p;
    a.g0 = mot0 & ~15u;  // f.p is 16-byte aligned
    a.fin = f.longueur;
    a.lds = lds;
    a.o2 = mot0 - a.g0;
    a.charge = OCTETS_ANNEAU / OCTETS_MORCEAU;
    a.limite = a.charge * OCTETS_MORCEAU - FENETRE;
    a.vol = u32x2{0u, 0u};
    a.en_vol = false;
    if (tuile) {
        const u32x2 d0 = lire_morceau_r(a, 0, v), d1 = lire_morceau_r(a, 1, v);
        const u32x2 d2 = lire_morceau_r(a, 2, v), d3 = lire_morceau_r(a, 3, v);
        ecrire_lds<u32x2>(lds + 0u * OCTETS_MORCEAU + v * 8u, d0);
        ecrire_lds<u32x2>(lds + 1u * OCTETS_MORCEAU + v * 8u, d1);
        ecrire_lds<u32x2>(lds + 2u * OCTETS_MORCEAU + v * 8u, d2);
        ecrire_lds<u32x2>(lds + 3u * OCTETS_MORCEAU + v * 8u, d3);
    }
    return a;
}

// End of a macro-step: land the chunk requested one macro-step ago (chunk charge - 1), request the
// next if due (the same schedule as avancer_anneau).
__device__ __forceinline__ void avancer_anneau_r(AnneauR& a, uint32_t v, bool actif) {
    if (a.en_vol) {
        ecrire_lds<u32x2>(a.lds + ((a.charge - 1u) & 3u) * OCTETS_MORCEAU + v * 8u, a.vol);
        a.en_vol = false;
    }
    if (actif && a.o2 > a.limite) {
        a.vol = lire_morceau_r(a, a.charge, v);
        a.charge += 1u;
        a.limite += OCTETS_MORCEAU;
        a.en_vol = true;
    }
}

// One decode step: LUT entry at lut + 8 (x mod 4096) (lut: LDS address of the context's table),
// the word of this lane at the half's pointer plus the renormalising lanes below it. Returns the
// entry's low word (f | s << 24). The ring pointer is advanced by the caller from `compte`.
template <bool TOUS_ACTIFS>
__device__ __forceinline__ uint32_t pas_r(uint32_t& x, uint32_t o2, uint32_t& compte, uint32_t lut, uint32_t anneau,
                                          uint32_t decal, uint32_t masque_inf, bool actif) {
    const u32x2 e = lire_lds<u32x2>(lut + ((x & (M - 1u)) << 3));
    const uint32_t y = __umul24(e.x, x >> PROBA_BITS) + e.y;
    const bool besoin = (TOUS_ACTIFS || actif) && (y < L);
    const uint64_t vote = __builtin_amdgcn_ballot_w64(besoin);
    const uint32_t moitie = uint32_t(vote >> decal);
    const uint32_t adr = ((o2 + 2u * (compte + __popc(moitie & masque_inf))) & (OCTETS_ANNEAU - 1u)) | anneau;
    const uint32_t w = lire_lds<uint16_t>(adr);
    const uint32_t suivant = besoin ? ((y << 16) | w) : y;
    x = (TOUS_ACTIFS || actif) ? suivant : x;
    compte += __popc(moitie);
    return e.x;
}

// `tete0`: premiere_tete(p.h), read by the caller before its barrier.
__device__ __forceinline__ void corps_gemv_rapide(const Tache& tc, const PrepGemv& p, uint8_t* lds,
                                                  uint32_t* __restrict__ controle, const TeteTuile& tete0) {
    const EnteteRans& h = p.h;
    const uint32_t R = tc.lignes, B = tc.colonnes / 32u, nblocs = R * B;
    const gptr<u32x4> ent16 = glob<u32x4>(reinterpret_cast<const void*>(tc.ech));
    float* __restrict__ partiels = reinterpret_cast<float*>(tc.partiels);
    const uint32_t kmax = tc.kmax;
    const uint32_t bpt = 8u * h.N;

    const uint32_t lane = __lane_id();
    const uint32_t v = lane & 31u;
    const bool haut = lane >= 32u;
    const uint32_t decal = haut ? 32u : 0u, masque_inf = (1u << v) - 1u;
    const uint32_t q = v >> 2, q4 = v & 3u;
    const uint32_t vagues_bloc = blockDim.x >> 6;
    // wave-uniform (scalar registers): the tile loop and its macro-step counts run on SALU
    const uint32_t vague = uniforme32(blockIdx.x * vagues_bloc + (threadIdx.x >> 6));
    const uint32_t n_vagues = gridDim.x * vagues_bloc;
    const uint32_t demi = (threadIdx.x >> 5) & (2u * vagues_bloc - 1u);
    const uint32_t base = adresse_lds(lds);
    const uint32_t a_lut = base + LDS_LUT;
    const uint32_t a_x = base + LDS_X + 16u * q4;          // | column offset from the entry
    const uint32_t a_anneau = base + LDS_ANNEAUX + demi * OCTETS_ANNEAU;
    const uint32_t a_ent = base + LDS_ENT + demi * (ENT_PAR_TUILE * 4u);
    const uint32_t a_ent_q = a_ent + 4u * q;
    // the stream header's counts, wave-uniform (scalar registers)
    const uint32_t hN = uniforme32(h.N), hT = uniforme32(h.T), nmacro = uniforme32(h.P / 128u);
    uint32_t hors_l = 0, pointeur = 0;
    TeteTuile tete = tete0;
    for (uint32_t t0 = 2u * vague; t0 < hT; t0 += 2u * n_vagues) {
        const uint32_t t = t0 + (haut ? 1u : 0u);
        const bool tuile = t < hT;
        const uint32_t nb_a = min(hN, nmacro - t0 * hN);
        const uint32_t nb_b = (t0 + 1u < hT) ? min(hN, nmacro - (t0 + 1u) * hN) : 0u;
        const uint32_t nb = haut ? nb_b : nb_a;
        const uint32_t m0 = (tuile ? t : t0) * hN;
        auto stager = [&](uint32_t m) { ecrire_lds<u32x4>(a_ent + 16u * v, ent16[2u * (m0 + m) + v]); };
        uint32_t x = tete.x;
        const uint32_t debut = tete.debut, attendu = tete.attendu;
        tete = lire_tete(h, t + 2u * n_vagues, v);
        if (tuile) stager(0);
        AnneauR a = ouvrir_anneau_r(h, p.fc, debut, a_anneau, v, tuile);
        const uint32_t o0 = a.o2;
        uint32_t rho = (m0 * 8u) / B;  // row of the tile's first block
        // partial slot of (row, t): rows that start inside tile t use slot 0, the tile's first row
        // (which may start in an earlier tile) its own offset, computed once
        const uint32_t rho0 = rho, case0 = t - premiere_tuile(rho0, B, bpt);
        auto ecrire = [&](float s) { ecrire_global<float>(partiels + rho * kmax + (rho == rho0 ? case0 : 0u), s); };
        uint32_t ent_suiv = tuile ? lire_lds<uint32_t>(a_ent_q) : ENTREE_BOURRAGE;
        const uint32_t nb_min = min(nb_a, nb_b);
        float acc = 0.0f;
        auto macro = [&](auto tous, uint32_t m) {
            constexpr bool TOUS = decltype(tous)::value;
            const bool actif = TOUS || m < nb;
            const uint32_t ent = actif ? ent_suiv : ENTREE_BOURRAGE;
            const uint32_t ax = (ent & ENT_X) | a_x;
            const f32x4 xa = lire_lds<f32x4>(ax);
            const f32x4 xb = lire_lds<f32x4>(ax + 64u);
            if (((m + 1u) & 15u) == 0u && m + 1u < (TOUS ? nb_min : nb)) stager(m + 1u);
            ent_suiv = lire_lds<uint32_t>(a_ent_q + 32u * ((m + 1u) & 15u));
            const uint32_t lt = a_lut + (ent & ENT_CTX);
            uint32_t compte = 0;
            const uint32_t e0 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            const uint32_t e1 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            const uint32_t e2 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            const uint32_t e3 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            a.o2 += 2u * compte;  // no vote in an inactive half: its pointer stays
            avancer_anneau_r(a, v, actif);
            // byte 3 of each LUT word is the decoded code byte: two E2M1 values, doubled by the 2.0
            // scale into the reference's k = {0,1,2,3,4,6,8,12} (exact)
            const f32x2 w0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e0, 2.0f, 3);
            const f32x2 w1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e1, 2.0f, 3);
            const f32x2 w2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e2, 2.0f, 3);
            const f32x2 w3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e3, 2.0f, 3);
            float d = w0.x * xa.x;
            d = fmaf(w0.y, xb.x, d);
            d = fmaf(w1.x, xa.y, d);
            d = fmaf(w1.y, xb.y, d);
            d = fmaf(w2.x, xa.z, d);
            d = fmaf(w2.y, xb.z, d);
            d = fmaf(w3.x, xa.w, d);
            d = fmaf(w3.y, xb.w, d);
            const float c = __builtin_amdgcn_ldexpf(d, int(ent << 7) >> 24);  // d * 2^(e-128), exact
            // a row starts in this macro-step (not the tile's own first row at its first block)
            const bool nouvelle = int(ent) < 0 && !(m == 0u && q == 0u && actif);
            const uint64_t vote = __builtin_amdgcn_ballot_w64(nouvelle);
            if (vote == 0) {
                if (TOUS || actif) acc += c;
            } else {
                // the half's first lane in the new row; lanes at or after it belong to row rho + 1
                const uint32_t moitie = uint32_t(vote >> decal);
                const uint32_t premier = moitie != 0u ? uint32_t(__builtin_ctz(moitie)) : 32u;
                const bool apres = v >= premier;
                if (!apres && (TOUS || actif)) acc += c;
                const float s = somme_demi_f32(acc);
                if (moitie != 0u) {
                    if (v == 0 && actif && rho < R) ecrire(s);
                    acc = apres ? c : 0.0f;
                    ++rho;
                }
            }
        };
        uint32_t m = 0;
        for (; m + 1u < nb_min; m += 2u) {  // two macro-steps per iteration: no register copies at the latch
            macro(std::true_type{}, m);
            macro(std::true_type{}, m + 1u);
        }
        if (m < nb_min) macro(std::true_type{}, m++);
        for (; m < nb_a; ++m) macro(std::false_type{}, m);
        const float s = somme_demi_f32(acc);
        if (tuile) {
            if (v == 0 && rho < R) ecrire(s);
            hors_l += (x != L) ? 1u : 0u;
            pointeur += (v == 0 && debut + (a.o2 - o0) / 2u != attendu) ? 1u : 0u;
        }
    }
    verser_controle(controle, hors_l, pointeur);
}

// --------------------------------------------------------------------------- row finishing

// What a finisher needs of a job: its biases, its partial sums and the tiles of each row.
struct Fin {
    const float* biais;
    const float* partiels;
    uint32_t kmax, B, bpt, lignes;
    uint32_t bon;
};

// The partial sums of row r after its first: tiles (rB + B - 1) / bpt - rB / bpt (shifts when the
// tiles hold a power-of-two number of blocks, as every CODES_CTX tile of 16 or 32 macro-steps does;
// the test is uniform).
__device__ __forceinline__ uint32_t partiels_en_plus(const Fin& f, uint32_t r) {
    const uint32_t a = r * f.B, b = a + f.B - 1u;
    if ((f.bpt & (f.bpt - 1u)) == 0u) {
        const uint32_t lg = uint32_t(__builtin_ctz(f.bpt));
        return (b >> lg) - (a >> lg);
    }
    return b / f.bpt - a / f.bpt;
}

// Whole wavefront (uniform job).
__device__ __forceinline__ Fin preparer_fin(const Tache& tc) {
    const MatricePartie m = obtenir_matrice(tc);
    const uint32_t B = tc.colonnes / 32u;
    Fin f;
    f.bon = m.bon != 0 && B >= 8u && (B - 1u) / (8u * m.cN) + 2u <= tc.kmax;
    f.biais = f.bon ? reinterpret_cast<const float*>(m.biais.p) : nullptr;
    f.partiels = reinterpret_cast<const float*>(tc.partiels);
    f.kmax = tc.kmax;
    f.B = B;
    f.bpt = f.bon ? 8u * m.cN : 1u;
    f.lignes = tc.lignes;
    return f;
}

// y[r] = fixed-order sum of row r's tile partials + bias[r].
__device__ __forceinline__ float somme_fin(const Fin& f, uint32_t r) {
    const uint32_t n = partiels_en_plus(f, r);
    const float* p = f.partiels + uint64_t(r) * f.kmax;
    float s = p[0];
    for (uint32_t k = 1; k <= n; ++k) s += p[k];
    return s + f.biais[r];
}

// Jobs first + y*par .. of the block parsed by one wavefront each, shared through LDS.
template <uint32_t N_MAX>
__device__ __forceinline__ void preparer_fins(const Taches& taches, uint32_t premier, uint32_t n, Fin (&fins)[N_MAX]) {
    const uint32_t w = threadIdx.x >> 6;
    for (uint32_t i = w; i < n; i += blockDim.x >> 6) {
        const Fin f = preparer_fin(uniforme(taches[premier + i]));
        if (__lane_id() == 0) fins[i] = f;
    }
    __syncthreads();
}


// gpt-oss clamped SwiGLU, the reference swiglu_oai's expression (passe.cuh:598-605): g <- min(g, 7),
// u <- clamp(u, -7, 7), g / (1 + exp(-1.702 g)) * (u + 1), evaluated in f32 with the device
// library's expf and IEEE division, a few ulp from the reference, which evaluates it in f64 and
// rounds once (the reference-API kernel swiglu_oai does that too). Every fused path (the down
// pass's prologue, fusion_finir_swiglu, the prefill's act pieces) takes this one, so their bits
// agree with each other.
__device__ __forceinline__ float swiglu_oai_f(float g, float u) {
    const float gv = fminf(g, 7.0f);
    const float uv = fminf(fmaxf(u, -7.0f), 7.0f);
    return gv / (1.0f + expf(-1.702f * gv)) * (uv + 1.0f);
}

}  // namespace trc
