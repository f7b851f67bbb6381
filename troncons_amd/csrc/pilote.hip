// pilote.hip — the driver half of the launch layer on HIP: context, streams, events, device memory,
// pinned and mapped host memory, asynchronous copies and fills, device attributes and the last
// error's HIP code. It replaces the hand-wrapped CUDA driver of the reference engine (the
// `trc_cuda` crate: Contexte, Flux, Evenement, MemoireCarte, HoteEpingle and the copies,
// moteur/crates/trc-cuda/src/lib.rs:160-623, over the entry points of api.rs:106-146), so that
// a caller owns every buffer and stream it hands to the Noyaux entry points without any other
// runtime.
//
// HIP has no explicit primary-context object: a trc_contexte names a device; every entry point
// that takes one makes its device current on the calling thread first (the reference makes its
// context current per thread, lazily, lib.rs:115-144). Streams and events are HIP handles passed
// as void*, exactly what every launch entry point takes as `flux`.
#include <hip/hip_runtime.h>

#include <cstring>
#include <string>

#include "erreurs.hpp"
#include "scratch.hpp"

struct trc_contexte {
    int ordinal = 0;
    uint32_t attente = 0;  // TRC_ATTENTE_* granted by the runtime
    char nom[256] = {};
    int version_pilote = 0;
};

namespace {

#define TRC_HIP_P(appel)                                                \
    do {                                                                \
        const hipError_t e_ = (appel);                                  \
        if (e_ != hipSuccess) return ::trc::erreur_hip(#appel, e_);     \
    } while (0)

int rendre_courant(const trc_contexte* c) {
    if (c == nullptr) return trc::usage("contexte nul");
    int d = -1;
    TRC_HIP_P(hipGetDevice(&d));
    if (d != c->ordinal) TRC_HIP_P(hipSetDevice(c->ordinal));
    return TRC_OK;
}

uint32_t drapeaux_attente(uint32_t attente) {
    switch (attente) {
        case TRC_ATTENTE_ACTIVE: return hipDeviceScheduleSpin;
        case TRC_ATTENTE_CEDE: return hipDeviceScheduleYield;
        case TRC_ATTENTE_BLOQUANTE: return hipDeviceScheduleBlockingSync;
        default: return hipDeviceScheduleAuto;
    }
}

uint32_t attente_de(unsigned drapeaux) {
    switch (drapeaux & hipDeviceScheduleMask) {
        case hipDeviceScheduleSpin: return TRC_ATTENTE_ACTIVE;
        case hipDeviceScheduleYield: return TRC_ATTENTE_CEDE;
        case hipDeviceScheduleBlockingSync: return TRC_ATTENTE_BLOQUANTE;
        default: return TRC_ATTENTE_AUTO;
    }
}

// One byte per thread, grid-stride (cuMemsetD8Async's job as a kernel, so that a caller capturing
// the stream into a graph records a kernel node rather than a memset node).
__global__ void __launch_bounds__(256) remplir_octets(uint8_t* __restrict__ p, uint64_t n, uint32_t mot) {
    const uint64_t i0 = (uint64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 16u;
    const uint64_t pas = uint64_t(gridDim.x) * blockDim.x * 16u;
    const bool aligne = (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
    for (uint64_t i = i0; i < n; i += pas) {
        if (aligne && i + 16u <= n) {
            *reinterpret_cast<uint4*>(p + i) = make_uint4(mot, mot, mot, mot);
        } else {
            for (uint64_t j = i; j < n && j < i + 16u; ++j) p[j] = uint8_t(mot);
        }
    }
}

}  // namespace

extern "C" {

// Contexte::nouveau_avec (lib.rs:166-201)
int trc_contexte_creer(uint32_t ordinal, uint32_t attente, trc_contexte** sortie) {
    if (sortie == nullptr) return trc::usage("sortie nulle");
    *sortie = nullptr;
    if (attente > TRC_ATTENTE_BLOQUANTE) return trc::usage("mode d'attente %u", attente);
    int n = 0;
    TRC_HIP_P(hipGetDeviceCount(&n));
    if (int(ordinal) >= n) return trc::usage("carte %u absente (%d cartes)", ordinal, n);
    TRC_HIP_P(hipSetDevice(int(ordinal)));
    // as with the primary context's flags: refused once the device is active, the runtime's stay
    (void)hipSetDeviceFlags(drapeaux_attente(attente));
    (void)hipGetLastError();
    // the library's per-device set-up: the allocation-free step's scratch address, so that a step
    // captured into a graph later makes no runtime query of its own
    const int rs = trc::preparer_scratch(int(ordinal));
    if (rs != TRC_OK) return rs;
    auto* c = new trc_contexte;
    c->ordinal = int(ordinal);
    unsigned d = 0;
    if (hipGetDeviceFlags(&d) == hipSuccess) c->attente = attente_de(d);
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, int(ordinal)) == hipSuccess) std::strncpy(c->nom, p.name, sizeof(c->nom) - 1);
    (void)hipDriverGetVersion(&c->version_pilote);
    *sortie = c;
    return TRC_OK;
}

void trc_contexte_detruire(trc_contexte* c) { delete c; }

// Contexte::memoire (lib.rs:204-213): (free, total) bytes of device memory
int trc_contexte_memoire(const trc_contexte* c, uint64_t* libre, uint64_t* totale) {
    if (libre == nullptr || totale == nullptr) return trc::usage("sorties nulles");
    const int r = rendre_courant(c);
    if (r != TRC_OK) return r;
    size_t l = 0, t = 0;
    TRC_HIP_P(hipMemGetInfo(&l, &t));
    *libre = l;
    *totale = t;
    return TRC_OK;
}

// Contexte::nom, version_pilote, attente_effective (lib.rs:215-232)
const char* trc_contexte_nom(const trc_contexte* c) { return c ? c->nom : ""; }
int trc_contexte_version_pilote(const trc_contexte* c) { return c ? c->version_pilote : 0; }
uint32_t trc_contexte_attente(const trc_contexte* c) { return c ? c->attente : 0; }

// Contexte::attribut (lib.rs:235-240, the attributes of lib.rs:251-276)
int trc_contexte_attribut(const trc_contexte* c, uint32_t attribut, int32_t* valeur) {
    if (valeur == nullptr) return trc::usage("sortie nulle");
    const int r = rendre_courant(c);
    if (r != TRC_OK) return r;
    hipDeviceAttribute_t a;
    switch (attribut) {
        case TRC_ATTRIBUT_CAPACITE_MAJEURE: a = hipDeviceAttributeComputeCapabilityMajor; break;
        case TRC_ATTRIBUT_CAPACITE_MINEURE: a = hipDeviceAttributeComputeCapabilityMinor; break;
        case TRC_ATTRIBUT_MOTEURS_DE_COPIE: a = hipDeviceAttributeAsyncEngineCount; break;
        case TRC_ATTRIBUT_PROJECTION_HOTE: a = hipDeviceAttributeCanMapHostMemory; break;
        case TRC_ATTRIBUT_ADRESSAGE_UNIFIE: a = hipDeviceAttributeUnifiedAddressing; break;
        case TRC_ATTRIBUT_UNITES_DE_CALCUL: a = hipDeviceAttributeMultiprocessorCount; break;
        case TRC_ATTRIBUT_LDS_PAR_BLOC: a = hipDeviceAttributeMaxSharedMemoryPerBlock; break;
        default: return trc::usage("attribut %u inconnu", attribut);
    }
    int v = 0;
    TRC_HIP_P(hipDeviceGetAttribute(&v, a, c->ordinal));
    *valeur = v;
    return TRC_OK;
}

// Contexte::synchroniser (lib.rs:243-246)
int trc_contexte_synchroniser(const trc_contexte* c) {
    const int r = rendre_courant(c);
    if (r != TRC_OK) return r;
    TRC_HIP_P(hipDeviceSynchronize());
    return TRC_OK;
}

// Flux::nouveau (lib.rs:290-302): non-blocking towards the null stream. Every stream gets the
// device's default priority: `priorite_haute` is accepted for the reference's signature only
// (streams of different priorities are not used on this platform).
int trc_flux_creer(const trc_contexte* c, int priorite_haute, void** flux) {
    (void)priorite_haute;
    if (flux == nullptr) return trc::usage("sortie nulle");
    *flux = nullptr;
    const int r = rendre_courant(c);
    if (r != TRC_OK) return r;
    hipStream_t s = nullptr;
    TRC_HIP_P(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *flux = s;
    return TRC_OK;
}

int trc_flux_detruire(void* flux) {
    if (flux == nullptr) return trc::usage("flux nul");
    TRC_HIP_P(hipStreamDestroy(reinterpret_cast<hipStream_t>(flux)));
    return TRC_OK;
}

// Flux::attendre (lib.rs:305-308): the stream waits for the event's last record
int trc_flux_attendre(void* flux, void* evenement) {
    if (flux == nullptr || evenement == nullptr) return trc::usage("flux ou evenement nul");
    TRC_HIP_P(hipStreamWaitEvent(reinterpret_cast<hipStream_t>(flux), reinterpret_cast<hipEvent_t>(evenement), 0));
    return TRC_OK;
}

// Flux::synchroniser (lib.rs:311-314)
int trc_flux_synchroniser(void* flux) {
    if (flux == nullptr) return trc::usage("flux nul");
    TRC_HIP_P(hipStreamSynchronize(reinterpret_cast<hipStream_t>(flux)));
    return TRC_OK;
}

// Flux::fini (lib.rs:318-326): 1 when every operation queued on the stream is over
int trc_flux_fini(void* flux, int* fini) {
    if (flux == nullptr || fini == nullptr) return trc::usage("flux ou sortie nuls");
    const hipError_t e = hipStreamQuery(reinterpret_cast<hipStream_t>(flux));
    if (e == hipErrorNotReady) {
        *fini = 0;
        return TRC_OK;
    }
    TRC_HIP_P(e);
    *fini = 1;
    return TRC_OK;
}

// Flux::priorite (lib.rs:329-331)
int trc_flux_priorite(void* flux, int* priorite) {
    if (flux == nullptr || priorite == nullptr) return trc::usage("flux ou sortie nuls");
    TRC_HIP_P(hipStreamGetPriority(reinterpret_cast<hipStream_t>(flux), priorite));
    return TRC_OK;
}

// Evenement::nouveau / nouveau_bloquant (lib.rs:361-379): `horodate` 0 disables timing
int trc_evenement_creer(const trc_contexte* c, int horodate, int bloquant, void** evenement) {
    if (evenement == nullptr) return trc::usage("sortie nulle");
    *evenement = nullptr;
    const int r = rendre_courant(c);
    if (r != TRC_OK) return r;
    unsigned d = (horodate ? hipEventDefault : hipEventDisableTiming) | (bloquant ? hipEventBlockingSync : 0u);
    hipEvent_t e = nullptr;
    TRC_HIP_P(hipEventCreateWithFlags(&e, d));
    *evenement = e;
    return TRC_OK;
}

int trc_evenement_detruire(void* evenement) {
    if (evenement == nullptr) return trc::usage("evenement nul");
    TRC_HIP_P(hipEventDestroy(reinterpret_cast<hipEvent_t>(evenement)));
    return TRC_OK;
}

// Evenement::enregistrer (lib.rs:382-385)
int trc_evenement_enregistrer(void* evenement, void* flux) {
    if (evenement == nullptr || flux == nullptr) return trc::usage("evenement ou flux nul");
    TRC_HIP_P(hipEventRecord(reinterpret_cast<hipEvent_t>(evenement), reinterpret_cast<hipStream_t>(flux)));
    return TRC_OK;
}

// Evenement::fini (lib.rs:388-396)
int trc_evenement_fini(void* evenement, int* fini) {
    if (evenement == nullptr || fini == nullptr) return trc::usage("evenement ou sortie nuls");
    const hipError_t e = hipEventQuery(reinterpret_cast<hipEvent_t>(evenement));
    if (e == hipErrorNotReady) {
        *fini = 0;
        return TRC_OK;
    }
    TRC_HIP_P(e);
    *fini = 1;
    return TRC_OK;
}

// Evenement::attendre (lib.rs:399-402)
int trc_evenement_attendre(void* evenement) {
    if (evenement == nullptr) return trc::usage("evenement nul");
    TRC_HIP_P(hipEventSynchronize(reinterpret_cast<hipEvent_t>(evenement)));
    return TRC_OK;
}

// Evenement::ms_depuis (lib.rs:406-414): milliseconds from `debut` to `fin`, both timed events
int trc_evenement_ms_depuis(void* fin, void* debut, float* ms) {
    if (fin == nullptr || debut == nullptr || ms == nullptr) return trc::usage("evenements ou sortie nuls");
    TRC_HIP_P(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(debut), reinterpret_cast<hipEvent_t>(fin)));
    return TRC_OK;
}

// MemoireCarte::allouer (lib.rs:448-458): the allocation as a view (hipMalloc: 256-byte aligned)
int trc_carte_allouer(const trc_contexte* c, uint64_t octets, trc_vue* vue) {
    if (vue == nullptr) return trc::usage("sortie nulle");
    *vue = trc_vue{0, 0};
    if (octets == 0) return trc::usage("allocation de VRAM de 0 octet");
    const int r = rendre_courant(c);
    if (r != TRC_OK) return r;
    void* p = nullptr;
    TRC_HIP_P(hipMalloc(&p, octets));
    *vue = trc_vue{uint64_t(reinterpret_cast<uintptr_t>(p)), octets};
    return TRC_OK;
}

// Drop for MemoireCarte (lib.rs:490-496): `vue` is what trc_carte_allouer gave
int trc_carte_liberer(const trc_contexte* c, trc_vue vue) {
    if (vue.adresse == 0) return trc::usage("vue nulle");
    const int r = rendre_courant(c);
    if (r != TRC_OK) return r;
    TRC_HIP_P(hipFree(reinterpret_cast<void*>(uintptr_t(vue.adresse))));
    return TRC_OK;
}

// MemoireCarte::remplir (lib.rs:481-487, cuMemsetD8Async): every byte of the view set to `octet`,
// asynchronously on `flux`, by a fill kernel
int trc_carte_remplir(trc_vue vue, uint8_t octet, void* flux) {
    if (vue.adresse == 0 && vue.octets != 0) return trc::usage("vue nulle");
    if (vue.octets == 0) return TRC_OK;
    const uint64_t groupes = (vue.octets + 16u * 256u - 1u) / (16u * 256u);
    const uint32_t g = uint32_t(groupes < 4096u ? groupes : 4096u);
    const uint32_t mot = uint32_t(octet) * 0x01010101u;
    hipLaunchKernelGGL(remplir_octets, dim3(g), dim3(256), 0, reinterpret_cast<hipStream_t>(flux),
                       reinterpret_cast<uint8_t*>(uintptr_t(vue.adresse)), vue.octets, mot);
    return trc::apres_lancement("remplir_octets");
}

// HoteEpingle::allouer (lib.rs:521-545): pinned, portable host memory, rounded up to 4096 bytes;
// with `projetee`, also mapped into the device's address space (its device address in *carte).
int trc_hote_allouer(const trc_contexte* c, uint64_t octets, int projetee, void** hote, uint64_t* octets_reels,
                     uint64_t* carte) {
    if (hote == nullptr) return trc::usage("sortie nulle");
    *hote = nullptr;
    if (octets == 0) return trc::usage("allocation epinglee de 0 octet");
    const int r = rendre_courant(c);
    if (r != TRC_OK) return r;
    const uint64_t n = (octets + 4095u) / 4096u * 4096u;
    void* p = nullptr;
    TRC_HIP_P(hipHostMalloc(&p, n, hipHostMallocPortable | (projetee ? hipHostMallocMapped : 0u)));
    if ((reinterpret_cast<uintptr_t>(p) & 4095u) != 0) {
        (void)hipHostFree(p);
        return trc::usage("hipHostMalloc a rendu une adresse non alignee sur 4096");
    }
    uint64_t d = 0;
    if (projetee) {
        void* dp = nullptr;
        const hipError_t e = hipHostGetDevicePointer(&dp, p, 0);
        if (e != hipSuccess) {
            (void)hipHostFree(p);
            return trc::erreur_hip("hipHostGetDevicePointer", e);
        }
        d = uint64_t(reinterpret_cast<uintptr_t>(dp));
    }
    *hote = p;
    if (octets_reels) *octets_reels = n;
    if (carte) *carte = d;
    return TRC_OK;
}

// Drop for HoteEpingle (lib.rs:582-588)
int trc_hote_liberer(void* hote) {
    if (hote == nullptr) return trc::usage("pointeur nul");
    TRC_HIP_P(hipHostFree(hote));
    return TRC_OK;
}

// HoteEpingle::lire_volatil_u32 (lib.rs:575-579): a u32 of mapped memory the device writes, read
// past the compiler's caching (a mailbox poll)
uint32_t trc_hote_lire_volatil_u32(const void* hote, uint64_t decalage) {
    return *reinterpret_cast<const volatile uint32_t*>(reinterpret_cast<const uint8_t*>(hote) + decalage);
}

// copier_vers_carte (lib.rs:591-603): `octets` bytes of pinned host memory at `src` into the view
int trc_copier_vers_carte(trc_vue dst, const void* src, uint64_t octets, void* flux) {
    if (src == nullptr || dst.adresse == 0) return trc::usage("source ou destination nulle");
    if (octets > dst.octets) return trc::usage("copie vers la carte : %llu octets dans une vue de %llu",
                                               (unsigned long long)octets, (unsigned long long)dst.octets);
    TRC_HIP_P(hipMemcpyAsync(reinterpret_cast<void*>(uintptr_t(dst.adresse)), src, octets, hipMemcpyHostToDevice,
                             reinterpret_cast<hipStream_t>(flux)));
    return TRC_OK;
}

// copier_vers_hote (lib.rs:606-614): the whole view into pinned host memory at `dst`
int trc_copier_vers_hote(void* dst, trc_vue src, void* flux) {
    if (dst == nullptr || src.adresse == 0) return trc::usage("source ou destination nulle");
    TRC_HIP_P(hipMemcpyAsync(dst, reinterpret_cast<const void*>(uintptr_t(src.adresse)), src.octets,
                             hipMemcpyDeviceToHost, reinterpret_cast<hipStream_t>(flux)));
    return TRC_OK;
}

// copier_carte_carte (lib.rs:617-623)
int trc_copier_carte_carte(trc_vue dst, trc_vue src, void* flux) {
    if (dst.adresse == 0 || src.adresse == 0) return trc::usage("source ou destination nulle");
    if (src.octets > dst.octets) return trc::usage("copie carte -> carte : la destination est plus courte que la source");
    TRC_HIP_P(hipMemcpyAsync(reinterpret_cast<void*>(uintptr_t(dst.adresse)),
                             reinterpret_cast<const void*>(uintptr_t(src.adresse)), src.octets,
                             hipMemcpyDeviceToDevice, reinterpret_cast<hipStream_t>(flux)));
    return TRC_OK;
}

}  // extern "C"
