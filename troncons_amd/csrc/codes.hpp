// codes.hpp — the CODES_CTX pass of the fused path with each CODES tile's DELTA decoded by the same
// half-wavefront right before it (gfx950). No block entry goes through device memory and no DELTA
// pass is launched.
//
// Streams of N_codes = 16 macro-steps per CODES tile: tile t covers blocks 128t .. 128t + 127, and
// its E8M0 scales and contexts are DELTA macro-step t. With N_delta = 1 that is DELTA tile t; with
// N_delta = 2 it is the first or second macro-step of DELTA tile t / 2 (the half-wavefront decodes
// that tile from its start). Everything a tile start needs from device memory is read one tile
// ahead into registers (Avance): the CODES lane states, the first 1 KiB of the CODES tile's words,
// the DELTA lane states and the first 512 bytes of its words, the row medians. At the tile start
// the half-wavefront
//   1. lands the DELTA words in its ring and decodes the DELTA macro-step(s) with the layer's
//      reference-format DELTA LUT (read through the L1: 4 to 8 steps per tile, against 64 CODES
//      steps), giving 4 delta bytes per lane (blocks 4v .. 4v + 3 of the tile);
//   2. turns them into the tile's 128 block entries (entree_bloc: e = (med + delta - 128) mod 256,
//      the context class of delta, column, row start) in its LDS entry area;
//   3. lands the CODES words in the ring (over the DELTA words) and decodes the tile as
//      corps_gemv_rapide does.
// A DELTA tile's end checks (every lane back to L, word pointer on the next tile's start) are made
// by the half-wavefront that decodes its last macro-step.
#pragma once

#include "fusion_corps.hpp"

namespace trc {

// A tile's streams read one tile ahead (per half-wavefront, lane v of the half).
struct Avance {
    TeteTuile tete;        // CODES: lane state, first word, word the decode must end on
    u32x4 mots0, mots1;    // CODES: bytes 16v and 512 + 16v of the tile's 16-aligned word area
    uint32_t xd;           // DELTA: lane state at the start of the DELTA tile
    uint32_t dDebut;       // DELTA: its first word
    uint32_t dAttendu;     // DELTA: the word its decode must end on
    u32x4 dmots;           // DELTA: bytes 16v of its 16-aligned word area (its first 512 bytes)
    uint32_t med0, med1;   // medians of the rows of blocks 4v and 4v + 3 of the CODES tile
    uint32_t rang0;        // the row of block 4v
    uint32_t med0b, med1b, rang0b;  // the same for blocks 128 + 4v .. of a tile of 32 macro-steps
};

// 16 bytes at byte `o` of a stream of `n` bytes (f.p 16-aligned), read at an address clamped to the
// stream's last 16-aligned 16 bytes: loads never leave the stream (the clamped lanes' bytes lie past
// the last word and are never decoded).
__device__ __forceinline__ u32x4 lire16_flux(const uint8_t* p, uint32_t n, uint32_t o) {
    const uint32_t dernier = n >= 16u ? ((n - 16u) & ~15u) : 0u;
    return *glob<u32x4>(p + min(o, dernier));
}

// Streams of CODES tile t (and, with DELTA, its DELTA tile) for lane v of a half-wavefront. Every
// load is unconditional, at an index clamped inside its stream (h.T >= 1): no branch surrounds
// them, so the compiler can count them, and a wait for an earlier load leaves these in flight. A
// tile past the stream reads the last tile's data, which its half never decodes nor checks.
// The CODES tile has hc.N = 16 or 32 macro-steps (128 or 256 blocks) and covers DELTA macro-steps
// hc.N / 16 * t .. (DELTA tile t / N_delta for 16, DELTA tile t for 32 with N_delta = 2).
template <bool DELTA>
__device__ __forceinline__ Avance lire_avance(const EnteteRans& hc, const DescFlux& fc, const EnteteRans& hd,
                                              const DescFlux& fd, const uint8_t* med, uint32_t R, const Diviseur& B,
                                              uint32_t t, uint32_t v) {
    Avance a;
    a.tete = lire_tete_borne(hc, t, v);
    const uint32_t base_c = uint32_t(reinterpret_cast<const uint8_t*>(hc.mots) - fc.p) + 2u * a.tete.debut;
    const uint32_t g0c = base_c & ~15u;
    a.mots0 = lire16_flux(fc.p, fc.longueur, g0c + 16u * v);
    a.mots1 = lire16_flux(fc.p, fc.longueur, g0c + 512u + 16u * v);
    a.xd = L;
    a.dDebut = a.dAttendu = 0;
    a.dmots = u32x4{0u, 0u, 0u, 0u};
    a.med0 = a.med1 = a.med0b = a.med1b = 0;
    a.rang0 = a.rang0b = 0;
    if (DELTA) {
        const uint32_t moitie = hc.N >> 5;  // 1 for tiles of 32 macro-steps
        const uint32_t tau = (t << moitie) >> (hd.N - 1u);  // N_delta being 1 or 2
        const TeteTuile td = lire_tete_borne(hd, tau, v);
        a.xd = td.x;
        a.dDebut = td.debut;
        a.dAttendu = td.attendu;
        const uint32_t base_d = uint32_t(reinterpret_cast<const uint8_t*>(hd.mots) - fd.p) + 2u * td.debut;
        a.dmots = lire16_flux(fd.p, fd.longueur, (base_d & ~15u) + 16u * v);
        // B >= 8: block 4v + 3 is in row rang0 or the next one
        const uint32_t bloc0 = ((128u * t) << moitie) + 4u * v;
        a.rang0 = B.quotient(bloc0);
        const uint32_t rang3 = a.rang0 + (bloc0 + 3u - a.rang0 * B.d >= B.d ? 1u : 0u);
        a.med0 = uint32_t(glob<uint8_t>(med)[min(a.rang0, R - 1u)]);
        a.med1 = uint32_t(glob<uint8_t>(med)[min(rang3, R - 1u)]);
        const uint32_t bloc0b = bloc0 + (moitie << 7);
        a.rang0b = B.quotient(bloc0b);
        const uint32_t rang3b = a.rang0b + (bloc0b + 3u - a.rang0b * B.d >= B.d ? 1u : 0u);
        a.med0b = uint32_t(glob<uint8_t>(med)[min(a.rang0b, R - 1u)]);
        a.med1b = uint32_t(glob<uint8_t>(med)[min(rang3b, R - 1u)]);
    }
    return a;
}

// One DELTA step with the reference-format LUT s | (f-1) << 8 | b << 20 read from device memory
// (its lines stay in the L1: every tile start of the block reads it), words from the ring.
// EN_LDS: the entry comes from the block's LDS copy at byte address `lutd_lds`, else from device
// memory.
template <bool TOUS_ACTIFS, bool EN_LDS>
__device__ __forceinline__ uint32_t pas_delta(uint32_t& x, uint32_t o2, uint32_t& compte, gptr<uint32_t> lutd,
                                              uint32_t lutd_lds, uint32_t anneau, uint32_t decal, uint32_t masque_inf,
                                              bool actif) {
    const uint32_t e = EN_LDS ? lire_lds<uint32_t>(lutd_lds + 4u * (x & (M - 1u))) : lutd[x & (M - 1u)];
    const uint32_t y = __umul24(((e >> 8) & 0xFFFu) + 1u, x >> PROBA_BITS) + (e >> 20);
    const bool besoin = (TOUS_ACTIFS || actif) && (y < L);
    const uint64_t vote = __builtin_amdgcn_ballot_w64(besoin);
    const uint32_t moitie = uint32_t(vote >> decal);
    const uint32_t adr = ((o2 + 2u * (compte + __popc(moitie & masque_inf))) & (OCTETS_ANNEAU - 1u)) | anneau;
    const uint32_t w = lire_lds<uint16_t>(adr);
    const uint32_t suivant = besoin ? ((y << 16) | w) : y;
    x = (TOUS_ACTIFS || actif) ? suivant : x;
    compte += __popc(moitie);
    return e & 0xFFu;
}

// Block entries of the CODES pass (LDS only; the separate DELTA pass keeps entree_bloc's layout):
//   bits 7-13   column block b (x byte offset b * 128 in LDS; 127 = the zero slot),
//   bits 15-16  context kappa (LUT byte offset kappa * 32 KiB),
//   bits 23-30  the block's biased E8M0 exponent e,
//   bit 31      the block starts a row.
// Read as an f32, an entry is +-(1.f) * 2^(e - 127). v_cvt_scalef32_pk_f32_fp4 takes only the
// exponent field of its scale operand (its sign and mantissa bits are ignored), so with the entry
// as scale it returns the block's weights E2M1 * 2^(e - 127) = k * 2^(e - 128) themselves, exact for
// e <= 252 (inf / NaN above). Padding: the zero slot with e = 127 (scale 1).
constexpr uint32_t ENTC_EXP = 23u;
constexpr uint32_t ENTC_BOURRAGE = (COLONNE_NULLE << 7) | (127u << ENTC_EXP);
// e - 128 of an entry (the scale of the tiles outside the scale-in-conversion range).
__device__ __forceinline__ int exposant_entree(uint32_t ent) { return int((ent ^ 0x40000000u) << 1) >> 24; }

// A lane's 4 entries (blocks 4v .. 4v + 3 of its CODES tile) and what its tile needs to know of them.
struct EntreesLane {
    u32x4 s;
    bool ligne;  // one of the 4 blocks starts a row (the tile's own first block excepted)
    uint32_t e4;  // the 4 blocks' E8M0 exponents e, block 4v + k in byte k (127 past the matrix)
    bool ech;    // every exponent e of the 4 lies in [64, 191]. The weights with the block scale
                 // folded in are then 2^(e-128) times the doubled E2M1 values, exactly, and every
                 // product and sum of the dot product with them is 2^(e-128) times the one without
                 // them, bit for bit, unless it leaves the normal f32 range (|x| beyond about 2^60
                 // or below 2^-60)
};

// The 4 block entries of lane v (blocks 4v .. 4v + 3 of a 128-block half of a CODES tile) from its
// 4 delta bytes, computed on packed bytes (byte k for block 4v + k) and gathered with byte permutes, no branch
// outside the stream's last tile:
//   e       = (med + delta - 128) mod 256, i.e. (med + delta) mod 256 with bit 7 flipped, added
//             byte-wise without carries between bytes, med being med0 (the median of row rang0,
//             block 4v's) up to the row's end and med1 after it (B >= 8: one row change at most);
//   kappa   = 0 below 128, 1 at 128, 2 above (bit 7 of delta, and an exact byte-wise zero test of
//             delta ^ 0x80);
//   column  = (4v + k - row start) per byte, the row start a byte-wise zero test of it.
// Byte k of the four packed values is entry k shifted right by 7: [column, kappa, e, row start].
__device__ __forceinline__ EntreesLane entrees_de_delta(uint32_t mot, uint32_t med0, uint32_t med1, uint32_t rang0,
                                                        uint32_t bloc0, uint32_t nblocs, const Diviseur& divB,
                                                        uint32_t masque_ligne) {
    const uint32_t B = divB.d;
    const uint32_t col0 = bloc0 - rang0 * B;
    const uint32_t reste = B - col0;  // blocks left in the row from block 4v (>= 1)
    const uint32_t apres = reste >= 4u ? 0u : (0xFFFFFFFFu << (8u * reste));  // bytes k >= reste
    const uint32_t medp = __builtin_amdgcn_perm(med1, med0, apres & 0x04040404u);
    uint32_t ee = ((medp & 0x7F7F7F7Fu) + (mot & 0x7F7F7F7Fu)) ^ ((medp ^ mot) & 0x80808080u) ^ 0x80808080u;
    const uint32_t vd = mot ^ 0x80808080u;
    const uint32_t nul = ~(((vd & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | vd | 0x7F7F7F7Fu);  // bit 7: delta byte == 128
    uint32_t kp = ((mot >> 6) & 0x02020202u) - (nul >> 7);
    uint32_t colp = __builtin_amdgcn_perm(0u, col0, 0x00000000u) + 0x03020100u - ((B * 0x01010101u) & apres);
    uint32_t rp = ~(((colp & 0x7F7F7F7Fu) + 0x7F7F7F7Fu) | colp | 0x7F7F7F7Fu) >> 7;  // 1 where the column is 0
    const uint32_t n_vrais = nblocs > bloc0 ? nblocs - bloc0 : 0u;
    if (n_vrais < 4u) {
        // blocks past the matrix: padding (the zero slot, context 0, e = 127, no row start)
        const uint32_t pad = 0xFFFFFFFFu << (8u * n_vrais);
        colp |= pad & 0x7F7F7F7Fu;
        kp &= ~pad;
        ee = (ee & ~pad) | (pad & 0x7F7F7F7Fu);
        rp &= ~pad;
    }
    EntreesLane r;
    r.e4 = ee;
    // e in [64, 191] <=> bits 7 and 6 of e differ
    r.ech = ((ee ^ (ee << 1)) & 0x80808080u) == 0x80808080u;
    r.ligne = (rp & masque_ligne) != 0u;
    const uint32_t lo = __builtin_amdgcn_perm(kp, colp, 0x05010400u), hi = __builtin_amdgcn_perm(kp, colp, 0x07030602u);
    const uint32_t lo2 = __builtin_amdgcn_perm(rp, ee, 0x05010400u), hi2 = __builtin_amdgcn_perm(rp, ee, 0x07030602u);
    r.s[0] = __builtin_amdgcn_perm(lo2, lo, 0x05040100u) << 7;
    r.s[1] = __builtin_amdgcn_perm(lo2, lo, 0x07060302u) << 7;
    r.s[2] = __builtin_amdgcn_perm(hi2, hi, 0x05040100u) << 7;
    r.s[3] = __builtin_amdgcn_perm(hi2, hi, 0x07060302u) << 7;
    return r;
}

// The launch's block size (a kernel's compile-time constant) and x-extent, the latter read once at
// kernel start into a scalar register: read later, after a barrier, it can come from a vector load
// of the dispatch packet whose wait would also drain the tile read-ahead in flight.
struct Grille {
    uint32_t fils, blocs_x;
};

// Tile lengths whose DELTA the CODES pass decodes itself: CODES tiles of 16 macro-steps with DELTA
// tiles of 1 or 2, or 32 with 2.
__host__ __device__ constexpr bool delta_dans_codes(uint32_t n_delta, uint32_t n_codes) {
    return (n_codes == 16u && (n_delta == 1u || n_delta == 2u)) || (n_codes == 32u && n_delta == 2u);
}

// What the CODES pass needs of a job in the internal-DELTA mode: both streams' headers, the
// medians, the DELTA LUT. bon: every check passed and the tile lengths are the mode's.
struct PrepCodes {
    DescFlux fc, fd;
    EnteteRans hc, hd;
    const uint8_t* med;
    Diviseur B;  // blocks per row
    bool bon;
};

__device__ __forceinline__ PrepCodes preparer_codes(const Tache& tc, const MatricePartie& m) {
    const uint32_t B = tc.colonnes / 32u;
    PrepCodes p;
    p.bon = m.bon != 0 && tc.colonnes % 32u == 0 && B >= 8u && tc.lignes > 0 &&
            delta_dans_codes(m.dN, m.cN) &&
            (B - 1u) / (8u * m.cN) + 2u <= tc.kmax;
    p.fc = m.codes;
    p.fd = m.delta;
    p.hc = entete_de(m.codes, m.cP, m.cN, m.cT, m.cW);
    p.hd = entete_de(m.delta, m.dP, m.dN, m.dT, m.dW);
    p.med = m.med.p;
    // the record carries the divider of B (computed once, where the record was made)
    p.B = m.div_m != 0u ? Diviseur{B, m.div_m, m.div_s & 255u, m.div_s >> 8} : Diviseur::de(B);
    return p;
}

// The first tile of the calling lane's half-wavefront (tile loops start at 2 * global wavefront).
template <bool DELTA>
__device__ __forceinline__ Avance premiere_avance(const PrepCodes& p, uint32_t R, const Grille& g) {
    const uint32_t vague = blockIdx.x * (g.fils >> 6) + (threadIdx.x >> 6);
    return lire_avance<DELTA>(p.hc, p.fc, p.hd, p.fd, p.med, R, p.B, 2u * vague + (__lane_id() >= 32u ? 1u : 0u),
                              __lane_id() & 31u);
}

// The DELTA stage of a tile pair, shared by the CODES pass and the slot decoder: the half's DELTA
// words landed in its ring, its DELTA macro-step(s) decoded (mot; mot_b: the second one of a tile
// of 32 macro-steps), the block's two first-tile barriers passed (premiere), the DELTA tile's end
// checks counted by the half that decoded its last macro-step.
struct ContexteDelta {
    gptr<uint32_t> lutd;  // the job's DELTA LUT (reference format) in device memory
    uint32_t a_lutd;      // its LDS copy (the entry area, for the first tiles)
    uint32_t a_anneau, decal, masque_inf, v;
    uint32_t mots_d;      // offset of the DELTA stream's words from its start
    uint32_t dN, dT, nmacro_d;
};

template <uint32_t NC>
__device__ __forceinline__ void delta_de_tuile(const PrepCodes& p, const ContexteDelta& cd, const Avance& cur,
                                               uint32_t t, bool tuile, bool& premiere, uint32_t& hors_l,
                                               uint32_t& pointeur, uint32_t& mot, uint32_t& mot_b) {
    const gptr<uint32_t> lutd = cd.lutd;
    const uint32_t a_lutd = cd.a_lutd, a_anneau = cd.a_anneau, decal = cd.decal, masque_inf = cd.masque_inf;
    const uint32_t v = cd.v, mots_d = cd.mots_d, dN = cd.dN, dT = cd.dT, nmacro_d = cd.nmacro_d;
    // NC = 16: the half's DELTA tile from its start to macro-step t mod N_delta (DELTA tile
    // t / N_delta covers CODES tiles t - t mod N_delta ..). NC = 32: DELTA tile t, both macro-steps.
    // Words from the ring.
    const uint32_t saut = NC == 32u ? 1u : (t & (dN - 1u));  // last DELTA macro-step needed
    const uint32_t saut_max = NC == 32u ? 1u : uniforme32(dN == 1u ? 0u : 1u);
    ecrire_lds<u32x4>(a_anneau + 16u * v, cur.dmots);
    {
        // two DELTA macro-steps can read up to 512 + 15 bytes: when the DELTA tile's words pass
        // the 512 read ahead (rare: about 50 bytes per macro-step here), the rest is read now
        const uint32_t o_d = (mots_d + 2u * cur.dDebut) & 15u;
        const bool long_d = tuile && o_d + 2u * (cur.dAttendu - cur.dDebut) > 512u;
        if (__builtin_amdgcn_ballot_w64(long_d) != 0) {
            const uint32_t g0d = (mots_d + 2u * cur.dDebut) & ~15u;
            const u32x4 suite = long_d ? lire16_flux(p.fd.p, p.fd.longueur, g0d + 512u + 16u * v)
                                       : u32x4{0u, 0u, 0u, 0u};
            if (long_d) ecrire_lds<u32x4>(a_anneau + 512u + 16u * v, suite);
        }
    }
    if (premiere) barriere_lds();  // the staged LUTs and x are visible
    const uint32_t tau = NC == 32u ? t : (t >> (dN - 1u));
    const uint32_t nbd = tau < dT ? min(dN, nmacro_d - tau * dN) : 0u;  // macro-steps of DELTA tile tau
    uint32_t xd = cur.xd, od = ((mots_d + 2u * cur.dDebut) & 15u);
    mot = 0;
    mot_b = 0;
    auto delta = [&](auto en_lds) {
        constexpr bool EN_LDS = decltype(en_lds)::value;
        for (uint32_t md = 0; md <= saut_max; ++md) {
            const bool actif = tuile && md <= saut && md < nbd;
            uint32_t compte = 0, m4 = 0;
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k)
                m4 |= pas_delta<false, EN_LDS>(xd, od, compte, lutd, a_lutd, a_anneau, decal, masque_inf, actif)
                      << (8u * k);
            od += 2u * compte;
            if (NC == 32u) {
                if (md == 0u) mot = m4;
                else mot_b = m4;
            } else if (md == saut) {
                mot = m4;
            }
        }
    };
    if (premiere)  // wave-uniform
        delta(std::true_type{});
    else
        delta(std::false_type{});
    if (premiere) {
        barriere_lds();  // no wave reads the DELTA LUT copy any more: the entry area is free
        premiere = false;
    }
    // the DELTA tile's end checks, by the half that decoded its last macro-step
    if (tuile && (NC == 32u ? nbd > 0u : saut + 1u == nbd)) {
        hors_l += (xd != L) ? 1u : 0u;
        pointeur += (v == 0 && cur.dDebut + (od - ((mots_d + 2u * cur.dDebut) & 15u)) / 2u != cur.dAttendu) ? 1u : 0u;
    }
}

// CODES_CTX tiles -> partial sums of W x, x in LDS, the tiles' entries decoded here from DELTA.
// `avance0`: premiere_avance(p), read by the caller. lutd: the job's DELTA LUT (reference format) in
// device memory. The caller stages the decode LUTs and x in LDS and, for the first tiles, a copy of
// the DELTA LUT over the entry area, without waiting: every wavefront passes the block's barrier
// before its first DELTA step (which reads that copy: an LDS read where the device-memory LUT would
// cost an L2 round trip per step, all waves waiting at once), and a second one before its first
// entries overwrite it. Later tiles read the DELTA LUT from device memory through the caches.
// NC: macro-steps per CODES tile, 16 (DELTA tiles of 1 or 2) or 32 (DELTA tiles of 2: CODES tile t
// is DELTA tile t). A tile of 32 keeps 128 entries in LDS like one of 16: the entries of its
// second 128 blocks are built with the first ones, held in registers, and written over slots that
// the tile has passed (lanes 0-15 at macro-step 8 for macro-steps 16-23, lanes 16-31 at
// macro-step 16 for 24-31); entry slot s serves macro-steps s and s + 16.
template <uint32_t NC>
__device__ __forceinline__ void corps_codes_n(const Tache& tc, const PrepCodes& p, uint8_t* lds,
                                              const uint32_t* lutd_, uint32_t* __restrict__ controle,
                                              const Avance& avance0, const Grille& g) {
    static_assert(NC == 16u || NC == 32u, "CODES tiles of 16 or 32 macro-steps");
    constexpr uint32_t BPT = 8u * NC;  // blocks per CODES tile
    const EnteteRans& h = p.hc;
    const EnteteRans& hd = p.hd;
    const uint32_t R = tc.lignes, B = tc.colonnes / 32u, nblocs = R * B;
    const gptr<uint32_t> lutd = glob<uint32_t>(lutd_);
    float* __restrict__ partiels = reinterpret_cast<float*>(tc.partiels);
    const uint32_t kmax = tc.kmax;

    const uint32_t lane = __lane_id();
    const uint32_t v = lane & 31u;
    const bool haut = lane >= 32u;
    const uint32_t decal = haut ? 32u : 0u, masque_inf = (1u << v) - 1u;
    const uint32_t q = v >> 2, q4 = v & 3u;
    const uint32_t vagues_bloc = g.fils >> 6;
    const uint32_t vague = uniforme32(blockIdx.x * vagues_bloc + (threadIdx.x >> 6));
    const uint32_t n_vagues = g.blocs_x * vagues_bloc;
    const uint32_t demi = (threadIdx.x >> 5) & (2u * vagues_bloc - 1u);
    const uint32_t base = adresse_lds(lds);
    const uint32_t a_lut = base + LDS_LUT;
    const uint32_t a_x = base + LDS_X + 16u * q4;
    const uint32_t a_anneau = base + LDS_ANNEAUX + demi * OCTETS_ANNEAU;
    const uint32_t a_ent = base + LDS_ENT + demi * (ENT_PAR_TUILE * 4u);
    const uint32_t a_ent_q = a_ent + 4u * q;
    const uint32_t hN = uniforme32(h.N), hT = uniforme32(h.T), nmacro = uniforme32(h.P / 128u);
    const uint32_t dN = uniforme32(hd.N), dT = uniforme32(hd.T), nmacro_d = uniforme32(hd.P / 128u);
    const uint32_t mots_c = uint32_t(reinterpret_cast<const uint8_t*>(h.mots) - p.fc.p);
    const uint32_t mots_d = uint32_t(reinterpret_cast<const uint8_t*>(hd.mots) - p.fd.p);
    uint32_t hors_l = 0, pointeur = 0;
    Avance av = avance0;
    bool premiere = true;  // wave-uniform: the block's two first-tile barriers are still to pass
    const uint32_t a_lutd = base + LDS_ENT;
    const ContexteDelta cd{lutd, a_lutd, a_anneau, decal, masque_inf, v, mots_d, dN, dT, nmacro_d};
    // the row-start bytes that count for `ligne`: all but the tile's own first block (lane 0, byte 0)
    const uint32_t masque_ligne = v == 0u ? 0x01010100u : 0x01010101u;
    // Issue priority by progress: a wavefront decodes its first tile pair at priority 3, then 2 from
    // the pair's middle macro-step, its second pair at 1 and then 0, so that on a SIMD the wavefronts
    // that are behind are issued ahead of those further on: their ends come closer together, and the
    // launch's tail (the last wavefronts running alone on their SIMDs) gets shorter.
    uint32_t paire_n = 0;
    __builtin_amdgcn_s_setprio(3);
    for (uint32_t t0 = 2u * vague; t0 < hT; t0 += 2u * n_vagues) {
        const uint32_t t = t0 + (haut ? 1u : 0u);
        const bool tuile = t < hT;
        const uint32_t nb_a = min(hN, nmacro - t0 * hN);
        const uint32_t nb_b = (t0 + 1u < hT) ? min(hN, nmacro - (t0 + 1u) * hN) : 0u;
        const uint32_t nb = haut ? nb_b : nb_a;
        const uint32_t m0 = (tuile ? t : t0) * hN;
        const Avance cur = av;

        // 1. DELTA
        uint32_t mot, mot_b;
        delta_de_tuile<NC>(p, cd, cur, t, tuile, premiere, hors_l, pointeur, mot, mot_b);
        // 2. the tile's block entries, which macro-steps start a row (macro-step m covers the
        // blocks of lanes 2m and 2m + 1: bit 2m of `lignes_m`, bit 2(m - 16) of `lignes_mb`), and
        // whether the wavefront's two tiles take the block scale inside the conversion
        const EntreesLane el = entrees_de_delta(mot, cur.med0, cur.med1, cur.rang0, BPT * t + 4u * v, nblocs, p.B,
                                                masque_ligne);
        if (tuile) ecrire_lds<u32x4>(a_ent + 16u * v, el.s);
        const uint64_t vl = __builtin_amdgcn_ballot_w64(tuile && el.ligne);
        uint32_t lignes_m = uint32_t(vl) | uint32_t(vl >> 32);
        lignes_m = (lignes_m | (lignes_m >> 1)) & 0x55555555u;
        bool ech_v = el.ech;
        u32x4 ent_b = u32x4{ENTC_BOURRAGE, ENTC_BOURRAGE, ENTC_BOURRAGE, ENTC_BOURRAGE};
        uint32_t lignes_mb = 0;
        if (NC == 32u) {
            const EntreesLane eb = entrees_de_delta(mot_b, cur.med0b, cur.med1b, cur.rang0b, BPT * t + 128u + 4u * v,
                                                    nblocs, p.B, 0x01010101u);
            ent_b = eb.s;
            const uint64_t vb = __builtin_amdgcn_ballot_w64(tuile && eb.ligne);
            lignes_mb = uint32_t(vb) | uint32_t(vb >> 32);
            lignes_mb = (lignes_mb | (lignes_mb >> 1)) & 0x55555555u;
            ech_v = ech_v && eb.ech;
        }
        const bool ech = __builtin_amdgcn_ballot_w64(tuile && !ech_v) == 0;
        // 3. the CODES words over the DELTA ones, and the next pair's streams read ahead
        ecrire_lds<u32x4>(a_anneau + 16u * v, cur.mots0);
        ecrire_lds<u32x4>(a_anneau + 512u + 16u * v, cur.mots1);
        av = lire_avance<true>(h, p.fc, hd, p.fd, p.med, R, p.B, t + 2u * n_vagues, v);
        AnneauR a;
        {
            const uint32_t mot0 = mots_c + 2u * cur.tete.debut;
            a.flux = p.fc.p;
            a.g0 = mot0 & ~15u;
            a.fin = p.fc.longueur;
            a.lds = a_anneau;
            a.o2 = mot0 - a.g0;
            a.charge = OCTETS_ANNEAU / OCTETS_MORCEAU;
            a.limite = a.charge * OCTETS_MORCEAU - FENETRE;
            a.vol = u32x2{0u, 0u};
            a.en_vol = false;
        }
        uint32_t x = cur.tete.x;
        const uint32_t debut = cur.tete.debut, attendu = cur.tete.attendu;
        const uint32_t o0 = a.o2;
        uint32_t rho = p.B.quotient(m0 * 8u);
        const uint32_t rho0 = rho, case0 = t - (rho0 * B) / BPT;  // first tile of row rho0
        // a global store: a flat one would also count on the LDS counter, and the next LUT read's
        // wait would then wait for the store's completion
        auto ecrire = [&](float s) { ecrire_global<float>(partiels + rho * kmax + (rho == rho0 ? case0 : 0u), s); };
        uint32_t ent_suiv = tuile ? lire_lds<uint32_t>(a_ent_q) : ENTC_BOURRAGE;
        const uint32_t nb_min = min(nb_a, nb_b);
        float acc = 0.0f;
        // One macro-step. TOUS: every lane of both halves active. ECH: the block scale inside the
        // conversion (the wavefront's entries are in the exact range). CONNUE: `ligne` says whether a
        // row starts in this macro-step (from lignes_m); otherwise the entries' row flags are voted.
        auto macro = [&](auto tous, auto echelle, auto connue, uint32_t m, bool ligne) {
            constexpr bool TOUS = decltype(tous)::value;
            constexpr bool ECH = decltype(echelle)::value;
            constexpr bool CONNUE = decltype(connue)::value;
            if (NC == 32u && (m == 8u || m == 16u)) {
                // the second 128 blocks' entries over the slots this tile has passed (wave-uniform test)
                if ((v < 16u) == (m == 8u) && tuile) ecrire_lds<u32x4>(a_ent + 16u * v, ent_b);
            }
            const bool actif = TOUS || m < nb;
            const uint32_t ent = actif ? ent_suiv : ENTC_BOURRAGE;
            const uint32_t ax = (ent & ENT_X) | a_x;
            const f32x4 xa = lire_lds<f32x4>(ax);
            const f32x4 xb = lire_lds<f32x4>(ax + 64u);
            ent_suiv = lire_lds<uint32_t>(a_ent_q + 32u * ((m + 1u) & 15u));
            const uint32_t lt = a_lut + (ent & ENT_CTX);
            uint32_t compte = 0;
            const uint32_t e0 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            const uint32_t e1 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            const uint32_t e2 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            const uint32_t e3 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            a.o2 += 2u * compte;
            avancer_anneau_r(a, v, actif);
            // byte 3 of each LUT word is the decoded code byte. ECH: scaled by the entry (its exponent
            // field is e), the weights themselves; otherwise doubled by 2.0 into the reference's
            // k = {0,1,2,3,4,6,8,12} and the dot product scaled by 2^(e-128) after. Both exact.
            const float sc = ECH ? __uint_as_float(ent) : 2.0f;
            const f32x2 w0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e0, sc, 3);
            const f32x2 w1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e1, sc, 3);
            const f32x2 w2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e2, sc, 3);
            const f32x2 w3 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(e3, sc, 3);
            float d = w0.x * xa.x;
            d = fmaf(w0.y, xb.x, d);
            d = fmaf(w1.x, xa.y, d);
            d = fmaf(w1.y, xb.y, d);
            d = fmaf(w2.x, xa.z, d);
            d = fmaf(w2.y, xb.z, d);
            d = fmaf(w3.x, xa.w, d);
            d = fmaf(w3.y, xb.w, d);
            const float c = ECH ? d : __builtin_amdgcn_ldexpf(d, exposant_entree(ent));
            // lanes whose block starts a row, except the tile's first block (lanes q == 0 of macro-step
            // 0 in each half): that row's sum goes to the tile's first slot. The entries of inactive
            // lanes are padding, which starts no row.
            auto voter = [&]() {
                return __builtin_amdgcn_ballot_w64(int(ent) < 0) & (m == 0u ? ~0x0000000F0000000Full : ~0ull);
            };
            uint64_t vote = 0;
            if (!CONNUE) vote = voter();
            // the sum with this macro-step's contribution, kept unless a row ends here
            float suite = (TOUS || actif) ? acc + c : acc;
            if (CONNUE ? ligne : vote != 0) {
                if (CONNUE) vote = voter();
                const uint32_t moitie = uint32_t(vote >> decal);
                const uint32_t premier = moitie != 0u ? uint32_t(__builtin_ctz(moitie)) : 32u;
                const bool apres = v >= premier;
                const float s = somme_demi_f32(apres ? acc : suite);
                if (moitie != 0u) {
                    if (v == 0 && actif && rho < R) ecrire(s);
                    suite = apres && (TOUS || actif) ? c : 0.0f;
                    ++rho;
                }
            }
            acc = suite;
        };
        const auto prio_milieu = [&]() {
            if (paire_n == 0u)
                __builtin_amdgcn_s_setprio(2);
            else
                __builtin_amdgcn_s_setprio(0);
        };
        // bit 2m of the row-start masks: macro-step m of the first 16 in lignes_m, of the next in lignes_mb
        const auto ligne_en = [&](uint32_t m) {
            return (((m < 16u ? lignes_m : lignes_mb) >> (2u * (m & 15u))) & 1u) != 0u;
        };
        if (nb_min == NC) {
            // both tiles whole (wave-uniform): macro-steps in pairs, the row starts known from the
            // entries (a scalar test per macro-step)
            auto tour = [&](auto echelle) {
#pragma unroll 1
                for (uint32_t mm = 0; mm < NC; mm += 2u) {
                    if (mm == NC / 2u) prio_milieu();
                    macro(std::true_type{}, echelle, std::true_type{}, mm, ligne_en(mm));
                    macro(std::true_type{}, echelle, std::true_type{}, mm + 1u, ligne_en(mm + 1u));
                }
            };
            if (ech)
                tour(std::true_type{});
            else
                tour(std::false_type{});
        } else {
            uint32_t m = 0;
            for (; m + 1u < nb_min; m += 2u) {
                if (m == NC / 2u) prio_milieu();
                macro(std::true_type{}, std::false_type{}, std::false_type{}, m, false);
                macro(std::true_type{}, std::false_type{}, std::false_type{}, m + 1u, false);
            }
            if (m < nb_min) macro(std::true_type{}, std::false_type{}, std::false_type{}, m++, false);
            for (; m < nb_a; ++m) macro(std::false_type{}, std::false_type{}, std::false_type{}, m, false);
        }
        const float s = somme_demi_f32(acc);
        if (tuile) {
            if (v == 0 && rho < R) ecrire(s);
            hors_l += (x != L) ? 1u : 0u;
            pointeur += (v == 0 && debut + (a.o2 - o0) / 2u != attendu) ? 1u : 0u;
        }
        if (paire_n == 0u)
            __builtin_amdgcn_s_setprio(1);
        else
            __builtin_amdgcn_s_setprio(0);
        ++paire_n;
    }
    if (premiere) {  // a wavefront without tiles still takes its part in both
        barriere_lds();
        barriere_lds();
    }
    verser_controle(controle, hors_l, pointeur);
}

// 4 scale bytes of blocks b0 .. b0 + 3 (b0 % 4 == 0) into a slot's 256-aligned scale array, those
// past the matrix left alone.
__device__ __forceinline__ void poser_echelles(uint8_t* ech, uint32_t b0, uint32_t e4, uint32_t nblocs, bool tuile) {
    if (!tuile || b0 >= nblocs) return;
    if (b0 + 4u <= nblocs) {
        ecrire_global<uint32_t>(reinterpret_cast<uint32_t*>(ech + b0), e4);
    } else {
        for (uint32_t k = 0; b0 + k < nblocs; ++k) ecrire_global<uint8_t>(ech + b0 + k, uint8_t(e4 >> (8u * k)));
    }
}

// The same tiles decoded into a slot instead of multiplied: CODES_CTX tiles of NC macro-steps, each
// with its DELTA decoded by its half-wavefront as in corps_codes_n (read one tile ahead, entries in
// LDS for the contexts), give the matrix's code bytes (codes, in stream order: the reference's
// [R][B][16 B]) and E8M0 scales (ech, [R][B]). The LDS regions are the CODES pass's (x unused).
// avance0: premiere_avance(p), read by the caller before it stages the LUTs.
template <uint32_t NC>
__device__ __forceinline__ void corps_codes_emplacement_n(const PrepCodes& p, uint32_t R, uint8_t* __restrict__ codes8,
                                                          uint8_t* __restrict__ ech, uint8_t* lds, const uint32_t* lutd_,
                                                          uint32_t* __restrict__ controle, const Avance& avance0,
                                                          const Grille& g) {
    static_assert(NC == 16u || NC == 32u, "CODES tiles of 16 or 32 macro-steps");
    constexpr uint32_t BPT = 8u * NC;
    const EnteteRans& h = p.hc;
    const EnteteRans& hd = p.hd;
    const uint32_t B = p.B.d, nblocs = R * B, mots_utiles = 4u * nblocs;
    uint32_t* __restrict__ codes = reinterpret_cast<uint32_t*>(codes8);
    const gptr<uint32_t> lutd = glob<uint32_t>(lutd_);
    const uint32_t lane = __lane_id();
    const uint32_t v = lane & 31u;
    const bool haut = lane >= 32u;
    const uint32_t decal = haut ? 32u : 0u, masque_inf = (1u << v) - 1u;
    const uint32_t q = v >> 2;
    const uint32_t vagues_bloc = g.fils >> 6;
    const uint32_t vague = uniforme32(blockIdx.x * vagues_bloc + (threadIdx.x >> 6));
    const uint32_t n_vagues = g.blocs_x * vagues_bloc;
    const uint32_t demi = (threadIdx.x >> 5) & (2u * vagues_bloc - 1u);
    const uint32_t base = adresse_lds(lds);
    const uint32_t a_lut = base + LDS_LUT;
    const uint32_t a_anneau = base + LDS_ANNEAUX + demi * OCTETS_ANNEAU;
    const uint32_t a_ent = base + LDS_ENT + demi * (ENT_PAR_TUILE * 4u);
    const uint32_t a_ent_q = a_ent + 4u * q;
    const uint32_t a_etage = base + LDS_X + demi * 512u;  // x's region: 32 halves x 4 macro-steps x 128 B
    const uint32_t hN = uniforme32(h.N), hT = uniforme32(h.T), nmacro = uniforme32(h.P / 128u);
    const uint32_t dN = uniforme32(hd.N), dT = uniforme32(hd.T), nmacro_d = uniforme32(hd.P / 128u);
    const uint32_t mots_c = uint32_t(reinterpret_cast<const uint8_t*>(h.mots) - p.fc.p);
    const uint32_t mots_d = uint32_t(reinterpret_cast<const uint8_t*>(hd.mots) - p.fd.p);
    uint32_t hors_l = 0, pointeur = 0;
    Avance av = avance0;
    bool premiere = true;  // wave-uniform: the block's two first-tile barriers are still to pass
    const ContexteDelta cd{lutd, base + LDS_ENT, a_anneau, decal, masque_inf, v, mots_d, dN, dT, nmacro_d};
    for (uint32_t t0 = 2u * vague; t0 < hT; t0 += 2u * n_vagues) {
        const uint32_t t = t0 + (haut ? 1u : 0u);
        const bool tuile = t < hT;
        const uint32_t nb_a = min(hN, nmacro - t0 * hN);
        const uint32_t nb_b = (t0 + 1u < hT) ? min(hN, nmacro - (t0 + 1u) * hN) : 0u;
        const uint32_t nb = haut ? nb_b : nb_a;
        const uint32_t m0 = (tuile ? t : t0) * hN;
        const Avance cur = av;
        uint32_t mot, mot_b;
        delta_de_tuile<NC>(p, cd, cur, t, tuile, premiere, hors_l, pointeur, mot, mot_b);
        // the entries (contexts) into LDS, the scales into the slot
        const EntreesLane el = entrees_de_delta(mot, cur.med0, cur.med1, cur.rang0, BPT * t + 4u * v, nblocs, p.B,
                                                0x01010101u);
        if (tuile) ecrire_lds<u32x4>(a_ent + 16u * v, el.s);
        poser_echelles(ech, BPT * t + 4u * v, el.e4, nblocs, tuile);
        u32x4 ent_b = u32x4{ENTC_BOURRAGE, ENTC_BOURRAGE, ENTC_BOURRAGE, ENTC_BOURRAGE};
        if (NC == 32u) {
            const EntreesLane eb = entrees_de_delta(mot_b, cur.med0b, cur.med1b, cur.rang0b, BPT * t + 128u + 4u * v,
                                                    nblocs, p.B, 0x01010101u);
            ent_b = eb.s;
            poser_echelles(ech, BPT * t + 128u + 4u * v, eb.e4, nblocs, tuile);
        }
        // the CODES words over the DELTA ones, and the next pair's streams read ahead
        ecrire_lds<u32x4>(a_anneau + 16u * v, cur.mots0);
        ecrire_lds<u32x4>(a_anneau + 512u + 16u * v, cur.mots1);
        av = lire_avance<true>(h, p.fc, hd, p.fd, p.med, R, p.B, t + 2u * n_vagues, v);
        AnneauR a;
        {
            const uint32_t mot0 = mots_c + 2u * cur.tete.debut;
            a.flux = p.fc.p;
            a.g0 = mot0 & ~15u;
            a.fin = p.fc.longueur;
            a.lds = a_anneau;
            a.o2 = mot0 - a.g0;
            a.charge = OCTETS_ANNEAU / OCTETS_MORCEAU;
            a.limite = a.charge * OCTETS_MORCEAU - FENETRE;
            a.vol = u32x2{0u, 0u};
            a.en_vol = false;
        }
        uint32_t x = cur.tete.x;
        const uint32_t debut = cur.tete.debut, attendu = cur.tete.attendu;
        const uint32_t o0 = a.o2;
        uint32_t ent_suiv = tuile ? lire_lds<uint32_t>(a_ent_q) : ENTC_BOURRAGE;
        const uint32_t nb_min = min(nb_a, nb_b);
        // GROUPE (both tiles whole): a macro-step's words go to the half's 512-byte staging area,
        // and every 4 macro-steps each lane stores 16 contiguous bytes of them (a quarter of the
        // global store instructions); otherwise each lane stores its word
        auto macro = [&](auto tous, auto groupe, uint32_t m) {
            constexpr bool TOUS = decltype(tous)::value;
            constexpr bool GROUPE = decltype(groupe)::value;
            if (NC == 32u && (m == 8u || m == 16u)) {
                // the second 128 blocks' entries over the slots this tile has passed (wave-uniform test)
                if ((v < 16u) == (m == 8u) && tuile) ecrire_lds<u32x4>(a_ent + 16u * v, ent_b);
            }
            const bool actif = TOUS || m < nb;
            const uint32_t ent = actif ? ent_suiv : ENTC_BOURRAGE;
            ent_suiv = lire_lds<uint32_t>(a_ent_q + 32u * ((m + 1u) & 15u));
            const uint32_t lt = a_lut + (ent & ENT_CTX);
            uint32_t compte = 0;
            const uint32_t e0 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            const uint32_t e1 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            const uint32_t e2 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            const uint32_t e3 = pas_r<TOUS>(x, a.o2, compte, lt, a_anneau, decal, masque_inf, actif);
            a.o2 += 2u * compte;
            avancer_anneau_r(a, v, actif);
            // byte 3 of each LUT word is the decoded code byte
            const uint32_t mot_c = __builtin_amdgcn_perm(e1, e0, 0x0C0C0703u) | __builtin_amdgcn_perm(e3, e2, 0x07030C0Cu);
            if (GROUPE) {
                ecrire_lds<uint32_t>(a_etage + 128u * (m & 3u) + 4u * v, mot_c);
                if ((m & 3u) == 3u) {
                    // lane v: words 4v .. 4v + 3 of the 4 macro-steps (macro-step v / 8, lanes 4 (v % 8) ..)
                    const u32x4 c = lire_lds<u32x4>(a_etage + 16u * v);
                    const uint32_t w = (m0 + m - 3u) * VOIES + 4u * v;
                    if (tuile && w < mots_utiles)  // read back by another launch: no reuse in the L2
                        ecrire_global_nt<u32x4>(codes + w, c);
                }
            } else {
                const uint32_t w = (m0 + m) * VOIES + v;
                if (actif && w < mots_utiles) ecrire_global<uint32_t>(codes + w, mot_c);
            }
        };
        if (nb_min == NC) {
#pragma unroll 1
            for (uint32_t mm = 0; mm < NC; mm += 2u) {
                macro(std::true_type{}, std::true_type{}, mm);
                macro(std::true_type{}, std::true_type{}, mm + 1u);
            }
        } else {
            uint32_t m = 0;
            for (; m < nb_min; ++m) macro(std::true_type{}, std::false_type{}, m);
            for (; m < nb_a; ++m) macro(std::false_type{}, std::false_type{}, m);
        }
        if (tuile) {
            hors_l += (x != L) ? 1u : 0u;
            pointeur += (v == 0 && debut + (a.o2 - o0) / 2u != attendu) ? 1u : 0u;
        }
    }
    if (premiere) {  // a wavefront without tiles still takes its part in both barriers
        barriere_lds();
        barriere_lds();
    }
    verser_controle(controle, hors_l, pointeur);
}

// The CODES pass for the job's tile length (uniform over the block: one matrix per block).
__device__ __forceinline__ void corps_codes(const Tache& tc, const PrepCodes& p, uint8_t* lds, const uint32_t* lutd_,
                                            uint32_t* __restrict__ controle, const Avance& avance0, const Grille& g) {
    if (uniforme32(p.hc.N) == 32u)
        corps_codes_n<32>(tc, p, lds, lutd_, controle, avance0, g);
    else
        corps_codes_n<16>(tc, p, lds, lutd_, controle, avance0, g);
}

}  // namespace trc
