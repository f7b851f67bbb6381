// anneau.hpp — LDS staging of a tile's renormalisation words and the 8-byte decode LUT of the fused
// path (gfx950).
//
// The words a tile's lanes read are consumed strictly in order, at most 32 per step. Each
// half-wavefront keeps its tile's words in a 1 KiB LDS ring made of two 512-byte chunks: while the
// read pointer is in chunk c, chunks c and c+1 are resident; when it enters c+1 (checked once per
// macro-step, which consumes at most 128 words = 256 bytes), chunk c+2 is loaded over chunk c with
// one 16-byte load per lane. A decode step therefore reads its word from LDS (one ds_read_u16)
// instead of waiting on a global load. Chunk loads never read past the end of the stream's
// descriptor (zeros beyond), so a corrupted stream cannot make a kernel read outside its part.
//
// The decode LUT is engine-internal (the reference's geometry-1 LUT s | (f-1)<<8 | b<<20 is what
// the host mounts; each block re-expands it into LDS): entry {f | s << 24, b}, so that
// y = f * (x >> 12) + b is one v_mad_u32_u24 (f <= 4096 sits in the low 24 bits).
#pragma once

#include "commun.hpp"

namespace trc {

// Global-address-space views: loads through them compile to global_load (vmcnt only) instead of
// flat_load (which also counts in lgkmcnt and would make every LDS wait wait for them too).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
template <typename T>
using gptr = __attribute__((address_space(1))) const T*;
template <typename T>
__device__ __forceinline__ gptr<T> glob(const void* p) {
    return (gptr<T>)(p);
}

constexpr uint32_t OCTETS_ANNEAU = 1024;
constexpr uint32_t OCTETS_MORCEAU = 512;

struct Anneau {
    const uint8_t* g0;   // 16-byte aligned global origin of the tile's words
    const uint8_t* fin;  // end of the stream: chunk loads never pass it
    uint32_t lds;        // byte offset of this half-wavefront's ring in the ring array
    uint32_t o2;         // byte offset from g0 of the next word to read (unwrapped)
    uint32_t charge;     // index of the next chunk to load
};

// Lane v (0..31) of the half-wavefront loads 16 bytes of chunk c into ring slot c & 1.
__device__ __forceinline__ void charger_morceau(const Anneau& a, uint8_t* anneaux, uint32_t c, uint32_t v) {
    const uint8_t* src = a.g0 + c * OCTETS_MORCEAU + v * 16u;
    u32x4 d = {0u, 0u, 0u, 0u};
    if (src + 16 <= a.fin) d = *glob<u32x4>(src);
    *reinterpret_cast<u32x4*>(anneaux + a.lds + (c & 1u) * OCTETS_MORCEAU + v * 16u) = d;
}

// Ring of tile t (words from mots + debut) at LDS offset `lds`; loads chunks 0 and 1.
__device__ __forceinline__ Anneau ouvrir_anneau(const EnteteRans& h, const DescFlux& f, uint32_t debut, uint32_t lds,
                                               uint8_t* anneaux, uint32_t v, bool tuile) {
    Anneau a;
    const uint8_t* mot0 = reinterpret_cast<const uint8_t*>(h.mots) + 2ull * debut;
    a.g0 = reinterpret_cast<const uint8_t*>(reinterpret_cast<uintptr_t>(mot0) & ~uintptr_t(15));
    a.fin = f.p + f.longueur;
    a.lds = lds;
    a.o2 = uint32_t(mot0 - a.g0);
    a.charge = 2;
    if (tuile) {
        charger_morceau(a, anneaux, 0, v);
        charger_morceau(a, anneaux, 1, v);
    }
    return a;
}

// After a macro-step: when the pointer has entered the newest resident chunk, refill the other.
__device__ __forceinline__ void avancer_anneau(Anneau& a, uint8_t* anneaux, uint32_t v, bool actif) {
    if (actif && (a.o2 / OCTETS_MORCEAU) + 1u >= a.charge) {
        charger_morceau(a, anneaux, a.charge, v);
        a.charge += 1u;
    }
}

// One decode step with the 8-byte LUT and the LDS ring; returns the LUT entry's low word
// (f | s << 24: the decoded byte is its top byte). `decal` is 0 for the lower half-wavefront and
// 32 for the upper one: the half's 32 ballot bits are one 64-bit shift away. ACTIF = false
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
__device__ __forceinline__ void etendre_luts(const uint32_t* __restrict__ src, uint2* dst, uint32_t n) {
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const uint32_t e = src[i];
        dst[i] = make_uint2((((e >> 8) & 0xFFFu) + 1u) | ((e & 0xFFu) << 24), e >> 20);
    }
}

}  // namespace trc
