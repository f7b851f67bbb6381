// anneau.hpp — LDS staging of a tile's renormalisation words and the 8-byte decode LUT of the fused
// path (gfx950).
//
// The words a tile's lanes read are consumed strictly in order, at most 32 per step and 128 per
// macro-step (256 bytes). Each half-wavefront keeps its tile's words in a 1 KiB LDS ring of four
// 256-byte chunks. Refills are software-pipelined by one macro-step so that a decode step never
// waits on device memory: at the end of a macro-step the chunk requested at the end of the previous
// one is written into the ring, then the next chunk is requested (one 8-byte load per lane, held
// in registers) if it starts less than 768 bytes past the read pointer. Invariant, given that a
// macro-step consumes at most 256 bytes: when a macro-step starts, every byte it can read is in
// LDS, and a chunk's slot is overwritten only after the pointer has left it. Chunk loads never
// read past the end of the stream's descriptor (zeros beyond), so a corrupted stream cannot make a
// kernel read outside its part.
//
// The decode LUT is engine-internal (the reference's geometry-1 LUT s | (f-1)<<8 | b<<20 is what
// the host mounts; each block re-expands it into LDS): entry {f | s << 24, b}, so that
// y = f * (x >> 12) + b is one v_mad_u32_u24 (f <= 4096 sits in the low 24 bits).
#pragma once

#include "commun.hpp"

namespace trc {

constexpr uint32_t OCTETS_ANNEAU = 1024;
constexpr uint32_t OCTETS_MORCEAU = 256;  // 8 bytes per lane of a half-wavefront
constexpr uint32_t FENETRE = 768;         // bytes past the read pointer that must be requested

struct Anneau {
    const uint8_t* g0;   // 16-byte aligned global origin of the tile's words
    const uint8_t* fin;  // end of the stream: chunk loads never pass it
    uint32_t lds;        // byte offset of this half-wavefront's ring in the ring array
    uint32_t o2;         // byte offset from g0 of the next word to read (unwrapped)
    uint32_t charge;     // index of the next chunk to request
    uint32_t c_vol;      // chunk held in `vol`
    u32x2 vol;           // this lane's 8 bytes of chunk c_vol, not yet in LDS
    bool en_vol;
};

__device__ __forceinline__ u32x2 lire_morceau(const Anneau& a, uint32_t c, uint32_t v) {
    const uint8_t* src = a.g0 + c * OCTETS_MORCEAU + v * 8u;
    u32x2 d = {0u, 0u};
    if (src + 8 <= a.fin) d = *glob<u32x2>(src);
    return d;
}

__device__ __forceinline__ void poser_morceau(const Anneau& a, uint8_t* anneaux, uint32_t c, uint32_t v, u32x2 d) {
    *reinterpret_cast<u32x2*>(anneaux + a.lds + (c & 3u) * OCTETS_MORCEAU + v * 8u) = d;
}

// Ring of tile t (words from mots + debut) at LDS offset `lds`; loads chunks 0-3.
__device__ __forceinline__ Anneau ouvrir_anneau(const EnteteRans& h, const DescFlux& f, uint32_t debut, uint32_t lds,
                                               uint8_t* anneaux, uint32_t v, bool tuile) {
    Anneau a;
    const uint8_t* mot0 = reinterpret_cast<const uint8_t*>(h.mots) + 2ull * debut;
    a.g0 = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(mot0) & ~uintptr_t(15));
    a.fin = f.p + f.longueur;
    a.lds = lds;
    a.o2 = uint32_t(mot0 - a.g0);
    a.charge = OCTETS_ANNEAU / OCTETS_MORCEAU;
    a.c_vol = 0;
    a.vol = u32x2{0u, 0u};
    a.en_vol = false;
    if (tuile) {
        const u32x2 d0 = lire_morceau(a, 0, v), d1 = lire_morceau(a, 1, v);
        const u32x2 d2 = lire_morceau(a, 2, v), d3 = lire_morceau(a, 3, v);
        poser_morceau(a, anneaux, 0, v, d0);
        poser_morceau(a, anneaux, 1, v, d1);
        poser_morceau(a, anneaux, 2, v, d2);
        poser_morceau(a, anneaux, 3, v, d3);
    }
    return a;
}

// End of a macro-step: land the chunk requested one macro-step ago, request the next if due.
__device__ __forceinline__ void avancer_anneau(Anneau& a, uint8_t* anneaux, uint32_t v, bool actif) {
    if (a.en_vol) {
        poser_morceau(a, anneaux, a.c_vol, v, a.vol);
        a.en_vol = false;
    }
    if (actif && a.charge * OCTETS_MORCEAU < a.o2 + FENETRE) {
        a.vol = lire_morceau(a, a.charge, v);
        a.c_vol = a.charge;
        a.charge += 1u;
        a.en_vol = true;
    }
}

// One decode step with the 8-byte LUT and the LDS ring; returns the LUT entry's low word
// (f | s << 24: the decoded byte is its top byte). `decal` is 0 for the lower half-wavefront and
// 32 for the upper one: the half's 32 ballot bits are one 64-bit shift away. TOUS_ACTIFS = false
// compiles the tail variant, where lanes past their tile's end keep their state.
template <bool TOUS_ACTIFS>
__device__ __forceinline__ uint32_t pas_anneau(uint32_t& x, Anneau& a, const uint2* __restrict__ lut,
                                               const uint8_t* __restrict__ anneaux, uint32_t decal,
                                               uint32_t masque_inf, bool actif) {
    const uint2 e = lut[x & (M - 1u)];
    const uint32_t y = __umul24(e.x, x >> PROBA_BITS) + e.y;
    const bool besoin = (TOUS_ACTIFS || actif) && (y < L);
    const uint64_t vote = __builtin_amdgcn_ballot_w64(besoin);
    const uint32_t moitie = uint32_t(vote >> decal);
    const uint32_t off = (a.o2 + 2u * __popc(moitie & masque_inf)) & (OCTETS_ANNEAU - 1u);
    const uint32_t w = *reinterpret_cast<const uint16_t*>(anneaux + a.lds + off);
    const uint32_t suivant = besoin ? ((y << 16) | w) : y;
    x = (TOUS_ACTIFS || actif) ? suivant : x;
    a.o2 += 2u * __popc(moitie);  // no vote in an inactive half: its pointer stays
    return e.x;
}

// Re-expands reference-format LUTs (s | (f-1)<<8 | b<<20) into 8-byte entries {f | s<<24, b}.
// n4 = number of 4-entry groups; every load of a batch is issued before the batch's stores.
__device__ __forceinline__ uint2 entree8(uint32_t e) {
    return make_uint2((((e >> 8) & 0xFFFu) + 1u) | ((e & 0xFFu) << 24), e >> 20);
}

template <uint32_t LOT>
__device__ __forceinline__ void etendre_luts(const uint32_t* __restrict__ src, uint2* dst, uint32_t n4,
                                             uint32_t debut = 0) {
    const gptr<u32x4> s4 = glob<u32x4>(src);
    for (uint32_t base = debut; base < n4; base += LOT * blockDim.x) {
        u32x4 t[LOT];
#pragma unroll
        for (uint32_t k = 0; k < LOT; ++k) {
            const uint32_t i = base + k * blockDim.x + threadIdx.x;
            if (i < n4) t[k] = s4[i];
        }
#pragma unroll
        for (uint32_t k = 0; k < LOT; ++k) {
            const uint32_t i = base + k * blockDim.x + threadIdx.x;
            if (i < n4) {
                uint2* d = dst + 4u * i;
                d[0] = entree8(t[k].x);
                d[1] = entree8(t[k].y);
                d[2] = entree8(t[k].z);
                d[3] = entree8(t[k].w);
            }
        }
    }
}

// The same in two halves, so that other loads are in flight meanwhile: demarrer() issues the first
// batch's loads, poser() stores them and expands the rest (blocks smaller than n4 / LOT threads).
// The first batch's loads are unconditional (index clamped; poser stores only the real ones): with
// no branch around them the compiler's wait counts stay exact, so waiting for a load issued before
// them does not also wait for them.
template <uint32_t LOT>
struct ChargeLut {
    u32x4 t[LOT];
    __device__ __forceinline__ void demarrer(const uint32_t* __restrict__ src, uint32_t n4) {
        const gptr<u32x4> s4 = glob<u32x4>(src);
#pragma unroll
        for (uint32_t k = 0; k < LOT; ++k) t[k] = s4[min(k * blockDim.x + threadIdx.x, n4 - 1u)];
    }
    __device__ __forceinline__ void poser(const uint32_t* __restrict__ src, uint2* dst, uint32_t n4) {
#pragma unroll
        for (uint32_t k = 0; k < LOT; ++k) {
            const uint32_t i = k * blockDim.x + threadIdx.x;
            if (i < n4) {
                uint2* d = dst + 4u * i;
                d[0] = entree8(t[k].x);
                d[1] = entree8(t[k].y);
                d[2] = entree8(t[k].z);
                d[3] = entree8(t[k].w);
            }
        }
        if (LOT * blockDim.x < n4) etendre_luts<LOT>(src, dst, n4, LOT * blockDim.x);
    }
};

// The three decode LUTs of a block of FILS threads (a compile-time size dividing 3 x 4096 / 4) in
// one batch of 3072 / FILS unconditional 16-byte loads per thread, expanded into LDS by poser():
// no loop and no branch, so the compiler's wait counts stay exact around them.
template <uint32_t FILS>
struct ChargeLutBloc {
    static constexpr uint32_t N4 = 3u * M / 4u;
    static constexpr uint32_t LOT = N4 / FILS;
    static_assert(N4 % FILS == 0, "the block size divides the LUT's 16-byte groups");
    u32x4 t[LOT];
    __device__ __forceinline__ void demarrer(const uint32_t* __restrict__ src) {
        const gptr<u32x4> s4 = glob<u32x4>(src);
#pragma unroll
        for (uint32_t k = 0; k < LOT; ++k) t[k] = s4[k * FILS + threadIdx.x];
    }
    __device__ __forceinline__ void poser(uint2* dst) const {
#pragma unroll
        for (uint32_t k = 0; k < LOT; ++k) {
            uint2* d = dst + 4u * (k * FILS + threadIdx.x);
            d[0] = entree8(t[k].x);
            d[1] = entree8(t[k].y);
            d[2] = entree8(t[k].z);
            d[3] = entree8(t[k].w);
        }
    }
};

// Copies n bytes (n <= cap) from device memory to LDS with 16-byte loads where the source allows
// it (src 16-byte aligned and the 16 bytes inside [src, src + lisible)), bytes otherwise.
__device__ __forceinline__ void copier_vers_lds(const uint8_t* src, uint32_t n, uint32_t lisible, uint8_t* dst) {
    const uint32_t n16 = (n + 15u) / 16u;
    for (uint32_t i = threadIdx.x; i < n16; i += blockDim.x) {
        if (16u * i + 16u <= lisible) {
            *reinterpret_cast<u32x4*>(dst + 16u * i) = *glob<u32x4>(src + 16u * i);
        } else {
            for (uint32_t k = 16u * i; k < n && k < 16u * i + 16u; ++k) dst[k] = glob<uint8_t>(src)[k];
        }
    }
}

}  // namespace trc
