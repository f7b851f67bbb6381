/*
 * troncons_hip.h — C-ABI of the MI355X (gfx950) expert hot path of troncons.
 *
 * Drop-in boundary: these entry points replace the CUDA launch layer of the reference engine,
 * i.e. the methods of `trc_noyaux::Noyaux` (moteur/crates/trc-noyaux/src/lib.rs) and the host
 * helpers of `trc_noyaux::abi` (moteur/crates/trc-noyaux/src/abi.rs). Arguments keep the
 * reference's order and meaning; each declaration cites the function it replaces. A Rust crate
 * binds them with `extern "C"`; nothing here uses torch or HIP types.
 *
 * Conventions (mirroring trc_cuda::Erreur, moteur/crates/trc-cuda/src/lib.rs:34-41):
 *   - every launch function returns TRC_OK, TRC_ERREUR_USAGE (a contract violation found before any
 *     HIP call: nothing was launched), TRC_ERREUR_HIP (a HIP call failed) or TRC_ERREUR_PILOTE (no
 *     usable device); trc_derniere_erreur() gives the message of the calling thread's last error;
 *   - launches are asynchronous on `flux` (a hipStream_t); data errors found by kernels are never
 *     returned: they are counted into the caller's zeroed u32[4] control buffer
 *     ([0] lanes not ending on L, [1] format errors, [2] tile word-pointer mismatches, [3] 0);
 *   - level-0 parts are 16-byte aligned (the device reader loads their header and descriptors 16
 *     bytes at a time; a misaligned part is a usage error, or a format error when its address is
 *     only known on the device);
 *   - the caller owns every allocation; a trc_vue borrows device memory for the call only.
 */
#ifndef TRONCONS_HIP_H
#define TRONCONS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TRC_OK 0
#define TRC_ERREUR_USAGE 1
#define TRC_ERREUR_HIP 2
#define TRC_ERREUR_PILOTE 3

/* VueCarte {u64 adresse; usize octets} (moteur/crates/trc-cuda/src/lib.rs:432-460): a device
 * address and a size in bytes. adresse == 0 stands for an absent optional view (Option::None). */
typedef struct {
    uint64_t adresse;
    uint64_t octets;
} trc_vue;

/* DimsExpert, 24 bytes, align 4 (abi.rs:8-13) */
typedef struct {
    uint32_t lignes[3];
    uint32_t colonnes[3];
} trc_dims_expert;

/* DescGemv, 32 bytes (abi.rs:18-27) */
typedef struct {
    uint64_t matrice;
    uint64_t x;
    uint64_t y;
    uint32_t lignes;
    uint32_t colonnes;
} trc_desc_gemv;

/* DescDecodage, 32 bytes (abi.rs:33-42) */
typedef struct {
    uint64_t partie;
    uint64_t emplacement;
    uint64_t luts;
    uint64_t controle;
} trc_desc_decodage;

/* Disposition of one matrix in the SoA slot (abi.rs:76-81) */
typedef struct {
    uint64_t base;
    uint64_t echelles;
    uint64_t biais;
    uint64_t pas;
} trc_disposition;

/* Message of the calling thread's last error ("" if none). */
const char* trc_derniere_erreur(void);

/* The hipError_t of the calling thread's last error when it was a HIP error (the `code` of
 * Erreur::Cuda, trc-cuda/src/lib.rs:34-41; its name and text are in trc_derniere_erreur()), else 0. */
int trc_dernier_code_hip(void);

/* ----------------------------------------------------- driver half (replaces the trc_cuda crate)
 *
 * Context, streams, events, device memory, pinned and mapped host memory, asynchronous copies and
 * fills on HIP, mirroring trc_cuda (moteur/crates/trc-cuda/src/lib.rs:160-623, api.rs:106-146).
 * A stream or an event is a HIP handle passed as void* (what every launch entry point takes as
 * `flux`). A trc_contexte names a device; each entry point that takes one makes its device current
 * on the calling thread first. Every stream is created at the device's default priority. */
typedef struct trc_contexte trc_contexte;

#define TRC_ATTENTE_AUTO 0      /* Attente::Auto (lib.rs:91-100): the runtime chooses */
#define TRC_ATTENTE_ACTIVE 1    /* Attente::Active: spin */
#define TRC_ATTENTE_CEDE 2      /* Attente::Cede: spin and yield */
#define TRC_ATTENTE_BLOQUANTE 3 /* Attente::Bloquante: the host thread sleeps */

#define TRC_ATTRIBUT_CAPACITE_MAJEURE 0 /* Attribut (lib.rs:251-276) */
#define TRC_ATTRIBUT_CAPACITE_MINEURE 1
#define TRC_ATTRIBUT_MOTEURS_DE_COPIE 2
#define TRC_ATTRIBUT_PROJECTION_HOTE 3
#define TRC_ATTRIBUT_ADRESSAGE_UNIFIE 4
#define TRC_ATTRIBUT_UNITES_DE_CALCUL 5 /* compute units (no counterpart in the reference) */
#define TRC_ATTRIBUT_LDS_PAR_BLOC 6     /* LDS bytes per workgroup (no counterpart in the reference) */

/* Contexte::nouveau_avec (lib.rs:166-201): device `ordinal` with host wait mode `attente`
 * (TRC_ATTENTE_*; kept by the runtime only if the device is not active yet). */
int trc_contexte_creer(uint32_t ordinal, uint32_t attente, trc_contexte** sortie);
void trc_contexte_detruire(trc_contexte* c);
/* Contexte::memoire (lib.rs:204-213): free and total device memory in bytes */
int trc_contexte_memoire(const trc_contexte* c, uint64_t* libre, uint64_t* totale);
/* Contexte::nom, version_pilote, attente_effective (lib.rs:215-232) */
const char* trc_contexte_nom(const trc_contexte* c);
int trc_contexte_version_pilote(const trc_contexte* c);
uint32_t trc_contexte_attente(const trc_contexte* c);
/* Contexte::attribut (lib.rs:235-240) */
int trc_contexte_attribut(const trc_contexte* c, uint32_t attribut, int32_t* valeur);
/* Contexte::synchroniser (lib.rs:243-246) */
int trc_contexte_synchroniser(const trc_contexte* c);

/* Flux::nouveau (lib.rs:290-302): a non-blocking stream; `priorite_haute` is accepted for the
 * signature, every stream gets the default priority. Drop for Flux (lib.rs:334-340). */
int trc_flux_creer(const trc_contexte* c, int priorite_haute, void** flux);
int trc_flux_detruire(void* flux);
/* Flux::attendre (lib.rs:305-308): `flux` waits for the last record of `evenement` */
int trc_flux_attendre(void* flux, void* evenement);
/* Flux::synchroniser (lib.rs:311-314) */
int trc_flux_synchroniser(void* flux);
/* Flux::fini (lib.rs:318-326): *fini = 1 when everything queued on the stream is over */
int trc_flux_fini(void* flux, int* fini);
/* Flux::priorite (lib.rs:329-331) */
int trc_flux_priorite(void* flux, int* priorite);

/* Evenement::nouveau / nouveau_bloquant (lib.rs:361-379); Drop for Evenement (lib.rs:417-423) */
int trc_evenement_creer(const trc_contexte* c, int horodate, int bloquant, void** evenement);
int trc_evenement_detruire(void* evenement);
/* Evenement::enregistrer (lib.rs:382-385) */
int trc_evenement_enregistrer(void* evenement, void* flux);
/* Evenement::fini (lib.rs:388-396) */
int trc_evenement_fini(void* evenement, int* fini);
/* Evenement::attendre (lib.rs:399-402) */
int trc_evenement_attendre(void* evenement);
/* Evenement::ms_depuis (lib.rs:406-414): milliseconds from `debut` to `fin` (timed events) */
int trc_evenement_ms_depuis(void* fin, void* debut, float* ms);

/* MemoireCarte::allouer (lib.rs:448-458) and its Drop (lib.rs:490-496): device memory as a view */
int trc_carte_allouer(const trc_contexte* c, uint64_t octets, trc_vue* vue);
int trc_carte_liberer(const trc_contexte* c, trc_vue vue);
/* MemoireCarte::remplir (lib.rs:481-487): every byte of `vue` set to `octet`, asynchronously on
 * `flux`, by a fill kernel (a graph capture of the stream records a kernel node) */
int trc_carte_remplir(trc_vue vue, uint8_t octet, void* flux);

/* HoteEpingle::allouer (lib.rs:521-545): pinned portable host memory rounded up to 4096 bytes
 * (*octets_reels), mapped into the device when `projetee` (its device address in *carte, else 0);
 * Drop for HoteEpingle (lib.rs:582-588) */
int trc_hote_allouer(const trc_contexte* c, uint64_t octets, int projetee, void** hote, uint64_t* octets_reels,
                     uint64_t* carte);
int trc_hote_liberer(void* hote);
/* HoteEpingle::lire_volatil_u32 (lib.rs:575-579): a mailbox word written by the device */
uint32_t trc_hote_lire_volatil_u32(const void* hote, uint64_t decalage);

/* copier_vers_carte, copier_vers_hote, copier_carte_carte (lib.rs:591-623): asynchronous on `flux`;
 * host memory is pinned memory from trc_hote_allouer */
int trc_copier_vers_carte(trc_vue dst, const void* src, uint64_t octets, void* flux);
int trc_copier_vers_hote(void* dst, trc_vue src, void* flux);
int trc_copier_carte_carte(trc_vue dst, trc_vue src, void* flux);

/* ------------------------------------------------------------- host helpers (no device needed) */

/* disposition_matrice (abi.rs:83-88) */
trc_disposition trc_disposition_matrice(uint32_t lignes, uint32_t colonnes);
/* DimsExpert::verifier (abi.rs:94-105): TRC_OK or TRC_ERREUR_USAGE */
int trc_dims_verifier(const trc_dims_expert* dims);
/* DimsExpert::disposition (abi.rs:108-111) */
trc_disposition trc_disposition_j(const trc_dims_expert* dims, uint32_t j);
/* DimsExpert::taille_emplacement (abi.rs:114-116) */
uint64_t trc_taille_emplacement(const trc_dims_expert* dims);
/* grilles_decodeur (abi.rs:137-141): grids (x, 3, 1) of decoder_echelles and decoder_codes */
void trc_grilles_decodeur(const trc_dims_expert* dims, uint32_t g_echelles[3], uint32_t g_codes[3]);
/* grilles_depuis_partie (abi.rs:149-176): grids sized on the tiles a part really has */
int trc_grilles_depuis_partie(const uint8_t* partie, size_t octets, uint32_t g_echelles[3], uint32_t g_codes[3]);
/* grille_brut (abi.rs:179-182) */
void trc_grille_brut(const trc_dims_expert* dims, uint32_t g[3]);
/* lut_geometrie1 (abi.rs:187-204): n must be 256, frequencies must sum to 4096 */
int trc_lut_geometrie1(const uint16_t* freq, size_t n, uint32_t* lut /* [4096] */);
/* luts_couche (abi.rs:210-221): freqs[j*4 + t] (t = 0 DELTA, 1 + kappa CODES_CTX) or NULL;
 * luts receives u32[3][4][4096] */
int trc_luts_couche(const uint16_t* const* freqs, uint32_t* luts);

/* ParamsRope (moteur/crates/trc-noyaux/src/abi.rs:229-251): YaRN parameters, 48 bytes; gpt-oss:
 * {150000, 32, 4096, 32, 1, 64, 0}. variante 0: OpenAI ramp bounds (the model); 1: llama.cpp's. */
typedef struct {
    double base, facteur, ctx_origine, beta_rapide, beta_lent;
    uint32_t dim_tete, variante;
} trc_params_rope;

/* ParamsAttention (abi.rs:253-291): one decode position's attention, 32 bytes. Positions
 * [debut, fin) are read; position pos lives in cache slot pos, or pos mod anneau when anneau > 0
 * (sliding-window layers). dim_tete must be 64; echelle = 1/sqrt(64). */
typedef struct {
    uint32_t tetes, tetes_kv, dim_tete, debut, fin, anneau;
    float echelle;
    uint32_t reserve;
} trc_params_attention;

#define TRC_ATTENTION_POSITIONS_MAX 8192 /* abi.rs:296-298 */

/* ---------------------------------------- launches: the reference kernel API (Noyaux methods) */

/* Noyaux::decoder_expert (moteur/crates/trc-noyaux/src/lib.rs:118-135): decodes a level-0 part
 * (v1.0/v1.2) into the SoA slot; two launches (scales, then codes) on flux. */
int trc_decoder_expert(trc_vue partie, trc_vue emplacement, trc_vue luts, const trc_dims_expert* dims,
                       trc_vue controle, void* flux);

/* Noyaux::decoder_expert_grilles (lib.rs:142-184): same with explicit grids (any grid is right). */
int trc_decoder_expert_grilles(trc_vue partie, trc_vue emplacement, trc_vue luts, const trc_dims_expert* dims,
                               trc_vue controle, const uint32_t g_echelles[3], const uint32_t g_codes[3], void* flux);

/* Noyaux::decoder_lot (lib.rs:190-205): n experts of the same dimensions, descs = DescDecodage[n]
 * in device memory. */
int trc_decoder_lot(trc_vue descs, uint32_t n, const trc_dims_expert* dims, void* flux);

/* Noyaux::copier_brut (lib.rs:210-233): raw-file path (flag bit 2). */
int trc_copier_brut(trc_vue partie, trc_vue emplacement, const trc_dims_expert* dims, trc_vue controle, void* flux);

/* Noyaux::gemv (lib.rs:239-268): y = W x + b for one slot matrix; bit-identical to the
 * reference's operation order (gemv.cuh:60-126). */
int trc_gemv(trc_vue matrice, trc_vue x, trc_vue y, uint32_t lignes, uint32_t colonnes, void* flux);

/* Noyaux::gemv_lot (lib.rs:274-284): n products from DescGemv[n] in device memory. */
int trc_gemv_lot(trc_vue descs, uint32_t n, uint32_t lignes_max, void* flux);

/* Noyaux::gemv_f32 (lib.rs:307-318): y = W x (+ b), W f32 row-major (the router). */
int trc_gemv_f32(trc_vue w, trc_vue x, trc_vue biais, trc_vue y, uint32_t lignes, uint32_t colonnes, void* flux);

/* Noyaux::routeur_topk (lib.rs:418-429): top-k indices and f64-softmax weights; boite = device
 * address of a mapped mailbox or 0 (words 1..k indices, k+1..2k weights, then word 0 = sequence,
 * written last after a system-scope fence). */
int trc_routeur_topk(trc_vue logits, uint32_t experts, uint32_t k, trc_vue indices, trc_vue poids, uint64_t boite,
                     uint32_t sequence, void* flux);

/* Noyaux::routeur_topk_biais (lib.rs:437-448, passe.cuh:516-580): the k chosen on logit + biais
 * (f32[experts]: beta for an expert already in VRAM), returned by unbiased logit with the softmax of
 * the unbiased logits; routeur_topk's bits when biais is zero. Same mailbox protocol. */
int trc_routeur_topk_biais(trc_vue logits, trc_vue biais, uint32_t experts, uint32_t k, trc_vue indices,
                           trc_vue poids, uint64_t boite, uint32_t sequence, void* flux);

/* Noyaux::swiglu_oai (lib.rs:451-458) */
int trc_swiglu_oai(trc_vue g, trc_vue u, trc_vue y, uint32_t n, void* flux);

/* Noyaux::combiner (lib.rs:463-476): residu[i] += ((w0 s0 + w1 s1) + w2 s2) + ..., no FMA. */
int trc_combiner(trc_vue residu, trc_vue sorties, uint32_t pas, trc_vue poids, uint32_t n, uint32_t d, void* flux);

/* ------------------------------------- launches: the fused path (extensions of the launch API)
 *
 * Added functions, nothing existing changed (the reference's own rule for extending its seam,
 * moteur/crates/trc-noyaux/noyaux/decodeur.cuh:227-231): the engine's caller of the expert hot
 * path is Modele::fin_couche (moteur/crates/trc-modele/src/lib.rs:533-553), which runs, per
 * selected expert, gemv(gate), gemv(up), swiglu_oai, gemv(down) over a decoded slot, then one
 * combiner. These entry points compute the same results from the coded part directly: the
 * decoded code bytes never reach device memory. `travail` is a caller-owned device workspace
 * (256-byte aligned) of at least the size the matching trc_taille_travail_* returns; n_delta and
 * n_codes are the macro-steps per tile of the DELTA and CODES_CTX streams (they size the grids
 * only: the kernels read the true N from every stream). Data errors go to `controle` as above. */

/* Workspace bytes of trc_gemv_fusionnee (0 if the shape is refused). */
uint64_t trc_taille_travail_gemv_fusionnee(uint32_t lignes, uint32_t colonnes, uint32_t n_codes);
/* Noyaux::decoder_expert + Noyaux::gemv for one matrix j of a part: y = W_j x + b_j. */
int trc_gemv_fusionnee(trc_vue partie, uint32_t j, trc_vue luts, uint32_t lignes, uint32_t colonnes, trc_vue x,
                       trc_vue y, trc_vue controle, trc_vue travail, uint32_t n_delta, uint32_t n_codes, void* flux);

/* Workspace bytes of trc_expert_fusionne. */
uint64_t trc_taille_travail_expert_fusionne(const trc_dims_expert* dims, uint32_t n_codes);
/* One expert of Modele::fin_couche (trc-modele/src/lib.rs:546-549):
 * sortie = W_down swiglu_oai(W_gate x + b_gate, W_up x + b_up) + b_down. */
int trc_expert_fusionne(trc_vue partie, trc_vue luts, const trc_dims_expert* dims, trc_vue x, trc_vue sortie,
                        trc_vue controle, trc_vue travail, uint32_t n_delta, uint32_t n_codes, void* flux);

/* Bytes of a layer directory for `experts` experts (3 entries of 128 bytes per expert). */
uint64_t trc_taille_repertoire(uint32_t experts);
/* Mounts a resident layer (no reference counterpart: the reference re-reads each part's header at
 * every decode, commun.cuh:101-165): parses the level-0 part of each expert once (parties:
 * u64[experts] device addresses of 16-byte aligned parts) into a device directory of stream
 * locations and checked headers, so that per-token launches do not walk the parts. A part that
 * fails a check counts one format error here and one more at each use. The parts must stay where
 * they are while the directory is used. */
int trc_monter_couche(trc_vue parties, uint32_t experts, const trc_dims_expert* dims, trc_vue repertoire,
                      trc_vue controle, void* flux);

/* ------------------------------- launches: the rest of the layer step (Noyaux, passe.cuh) */

/* Noyaux::gemv_q8_0 (lib.rs:291-302): y = W x (+ biais), W Q8_0 (rows of colonnes/32 blocks of 34
 * bytes: f16 d, 32 x i8), in the reference's operation order (lane l of 32 takes blocks l, l + 32,
 * ...; butterfly). w 2-byte aligned, x 16-byte aligned; biais may be absent (adresse 0). */
int trc_gemv_q8_0(trc_vue w, trc_vue x, trc_vue biais, trc_vue y, uint32_t lignes, uint32_t colonnes, void* flux);
/* Noyaux::ligne_q8_0 (lib.rs:478-486): row `ligne` of a Q8_0 matrix (the embedding) -> f32, exact. */
int trc_ligne_q8_0(trc_vue w, uint32_t ligne, uint32_t colonnes, trc_vue y, void* flux);
/* Noyaux::rmsnorm (lib.rs:322-330): `lignes` rows of n, y = x * r * w with r = 1/sqrt(mean(x^2) +
 * eps), sums and products in f64 (fixed tree), rounded once; y may equal x. */
int trc_rmsnorm(trc_vue x, trc_vue w, trc_vue y, uint32_t n, uint32_t lignes, float eps, void* flux);
/* Noyaux::rope_yarn (lib.rs:334-343): NEOX YaRN rotation of tetes_q heads of q and tetes_k heads
 * of k, in place, at `position`, in f64. */
int trc_rope_yarn(trc_vue q, trc_vue k, uint32_t tetes_q, uint32_t tetes_k, uint32_t position,
                  const trc_params_rope* p, void* flux);
/* Noyaux::ecrire_kv (lib.rs:348-357): k, v (f32[dkv]) rounded to f16 (nearest even) into slot
 * case_kv of the layer's caches ([slot][kv head][64]). */
int trc_ecrire_kv(trc_vue k, trc_vue v, trc_vue cache_k, trc_vue cache_v, uint32_t dkv, uint32_t case_kv, void* flux);
/* Noyaux::attention (lib.rs:362-379): decode attention of one position, every query head, with
 * the per-head sinks in the softmax denominator; puits f32[tetes], sortie f32[tetes * 64]. */
int trc_attention(trc_vue q, trc_vue cache_k, trc_vue cache_v, trc_vue puits, trc_vue sortie,
                  const trc_params_attention* p, void* flux);

/* Noyaux::ecrire_kv_f32 / attention_kvf32 (lib.rs:383-411, passe.cuh:374-445): the trial f32 KV
 * cache: k and v stored unrounded, then the same attention arithmetic in the same order (the
 * f16 path's bits whenever the keys and values are exact in f16). Cache views: f32[cases][dkv]. */
int trc_ecrire_kv_f32(trc_vue k, trc_vue v, trc_vue cache_k, trc_vue cache_v, uint32_t dkv, uint32_t case_kv,
                      void* flux);
int trc_attention_kvf32(trc_vue q, trc_vue cache_k, trc_vue cache_v, trc_vue puits, trc_vue sortie,
                        const trc_params_attention* p, void* flux);
/* Noyaux::argmax (lib.rs:490-496): index of the largest of n floats (ties: lower index; NaN never
 * chosen; all NaN: 0xFFFFFFFF) into sortie (u32). */
int trc_argmax(trc_vue v, uint32_t n, trc_vue sortie, void* flux);

/* ------------------------------------------------ the decode step of a model (trc_modele::Modele) */

/* Hyper (trc-modele/src/lib.rs:60-79): a gpt-oss-shaped model; heads of 64 (rope.dim_tete = 64);
 * even layers are windowed on a ring of `fenetre` positions, odd ones keep `contexte` positions. */
typedef struct {
    uint32_t couches, d, tetes, tetes_kv, experts, actifs, vocab, fenetre, contexte, n_delta, n_codes;
    float eps;
    trc_params_rope rope;
    trc_dims_expert dims;
} trc_hyper;

/* One layer's device views, owned by the caller (Modele's CoucheResidente, lib.rs:300-360):
 * attention weights in Q8_0 and f32, the sinks, the router (bf16, experts x d, 8-byte aligned) and
 * its optional bias, the layer's mounted directory (trc_monter_couche) and LUTs, the f16 KV caches
 * (ring of fenetre slots on even layers, contexte slots on odd ones). */
typedef struct {
    trc_vue attn_norm, wq, bq, wk, bk, wv, bv, wo, bo, puits, post_norm;
    trc_vue routeur, routeur_biais, repertoire, luts, cache_k, cache_v;
} trc_couche_modele;

typedef struct trc_modele trc_modele;

/* Workspace bytes of trc_modele_creer (0 if the shape is refused). */
uint64_t trc_modele_taille_travail(const trc_hyper* h);
/* Modele::charger's device side (lib.rs:366-455) over resident weights: keeps the views and cuts
 * `travail` (256-aligned) into the step's buffers. The caller keeps every view alive. */
int trc_modele_creer(const trc_hyper* h, const trc_couche_modele* couches, trc_vue enchassement,
                     trc_vue norme_sortie, trc_vue sortie, trc_vue travail, trc_modele** m);
void trc_modele_detruire(trc_modele* m);
/* Views of the residual x, the logits (f32[vocab]), the greedy token (u32), the last layer's
 * top-k indices (u32[8]) and the control words (u32[4], to be zeroed by the caller). */
int trc_modele_vues(const trc_modele* m, trc_vue* x, trc_vue* logits, trc_vue* jeton, trc_vue* indices,
                    trc_vue* controle);
/* Modele::enchasser (lib.rs:481-487): x = row `jeton` of the Q8_0 embedding. */
int trc_modele_enchasser(trc_modele* m, uint32_t jeton, void* flux);
/* Layer l at `position`: Modele::debut_couche (lib.rs:498-530) with the router and
 * Modele::fin_couche (lib.rs:533-555) as one fused compressed MoE layer. */
int trc_modele_couche(trc_modele* m, uint32_t l, uint32_t position, void* flux);
/* Modele::sortie (lib.rs:557-568): output norm, Q8_0 logits, argmax. */
int trc_modele_sortie(trc_modele* m, void* flux);
/* One decode step: enchasser, every layer, sortie (asynchronous on flux, no host sync). */
int trc_modele_pas(trc_modele* m, uint32_t jeton, uint32_t position, void* flux);

/* Workspace bytes of trc_couche_moe_fusionnee. */
uint64_t trc_taille_travail_couche_moe(const trc_dims_expert* dims, uint32_t experts, uint32_t k, uint32_t n_codes);
/* One MoE layer step at batch 1 (Modele::debut_couche's router, gemv_f32 + routeur_topk, then
 * Modele::fin_couche): logits = routeur x (+ routeur_biais) with a bf16 experts x C router, top-k
 * and softmax weights (written to indices / poids), the k fused experts, and
 * residu[i] += ((w0 s0[i] + w1 s1[i]) + ...). repertoire: the layer's directory
 * (trc_monter_couche); the selection never leaves the device. */
int trc_couche_moe_fusionnee(trc_vue repertoire, uint32_t experts, trc_vue luts, const trc_dims_expert* dims,
                             trc_vue routeur, trc_vue routeur_biais, trc_vue x, uint32_t k, trc_vue residu,
                             trc_vue indices, trc_vue poids, trc_vue controle, trc_vue travail, uint32_t n_delta,
                             uint32_t n_codes, void* flux);

/* No counterpart in the reference. For callers that cannot allocate (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): trc_couche_moe_fusionnee with the library's
 * static device scratch (trc_octets_scratch() bytes, 16 MiB, one per device, held until the process
 * ends) as its workspace; it calls no allocating routine. A step needing more than the scratch
 * (trc_taille_travail_couche_moe) is a usage error. Every call on a device shares that device's
 * scratch: calls that overlap on one device (two streams, two threads) race; serialise them. The
 * scratch is taken on the device of `flux` (the current device if flux is null); its device address
 * is resolved once per device, by trc_contexte_creer (the library's set-up of a device) or else at
 * the first call there. A caller that captures the step into a HIP graph creates the device's
 * context, or makes one call, before the capture: the captured call then makes no runtime query. */
uint64_t trc_octets_scratch(void);
int trc_couche_moe_fusionnee_sans_alloc(trc_vue repertoire, uint32_t experts, trc_vue luts,
                                        const trc_dims_expert* dims, trc_vue routeur, trc_vue routeur_biais,
                                        trc_vue x, uint32_t k, trc_vue residu, trc_vue indices, trc_vue poids,
                                        trc_vue controle, uint32_t n_delta, uint32_t n_codes, void* flux);

/* Workspace bytes of trc_prefill_moe (0 if the shape is refused). */
uint64_t trc_taille_travail_prefill(const trc_dims_expert* dims, uint32_t experts, uint32_t positions, uint32_t k,
                                    uint32_t n_codes);
/* Batched prefill of one resident MoE layer: replaces the per-layer expert part of the reference's
 * prefill, trc-ordo/src/lib.rs:814-941 (par_expert grouping of the positions' top-k, one decode per
 * chosen expert, Modele::expert_pos per (position, slot) and Modele::combiner_pos per position,
 * trc-modele/src/lib.rs:688-710). x: f32[positions][C]; indices / poids: u32 / f32 [positions][k]
 * (the routers' output, debut_couche_pos); residus: f32[positions][D], residus[i] += ((w_i0 s_i0 +
 * w_i1 s_i1) + ...). Each chosen expert is decoded once, into LDS, and applied to all its positions
 * on the bf16 MFMA (MXFP4 weights are exact in bf16; x and the SwiGLU rows are split into exact bf16
 * pieces); rows of at most 4096 columns. Tiles of at most 16 macro-steps (n_codes <= 16) are decoded
 * band by band straight into LDS; longer ones (the reference encoder's 256) are first decoded once
 * per chosen expert into a slot of the workspace, from which the bands are copied. An index >=
 * experts counts one format error and leaves its position alone. */
int trc_prefill_moe(trc_vue repertoire, uint32_t experts, trc_vue luts, const trc_dims_expert* dims, trc_vue x,
                    uint32_t positions, trc_vue indices, trc_vue poids, uint32_t k, trc_vue residus,
                    trc_vue controle, trc_vue travail, uint32_t n_delta, uint32_t n_codes, void* flux);

/* Chronogram of the fused entry points (role of the reference's --chronogramme, which records GPU
 * event timestamps around each decode, moteur/crates/trc-ordo/src/lib.rs:205-222): off by
 * default; when on, every kernel a fused entry point launches is bracketed by two HIP events on
 * its stream. trc_chrono_recolter waits for the recorded pairs and copies out at most `max`
 * (name[64], total ms, launches) entries; returns the number of names. */
void trc_chrono(int actif);
int trc_chrono_recolter(char* noms, double* ms, uint64_t* lancements, int max, int remettre_a_zero);

/* ------------------------------------------- the .trc v1.2 file container (host only; trc-format)
 *
 * Replaces the Rust crate trc-format (moteur/crates/trc-format/src/lib.rs) for the scheduler's
 * side of the path: Fichier::ouvrir and its accessors (lib.rs:957-1140), lire_partie
 * (lib.rs:813-866), assembler_partie (lib.rs:879-910), the Ecrivain (lib.rs:1149-1239) and
 * empreinte64 (lib.rs:111-127). The reader refuses what the reference refuses; its status codes
 * are the classes of ErreurFormat (lib.rs:129-148), with the message in trc_derniere_erreur(). */

#define TRC_FORMAT_ES 16        /* read/write error, short file */
#define TRC_FORMAT_MAGIE 17     /* not a .trc file */
#define TRC_FORMAT_VERSION 18   /* major != 1 or minor > 2 */
#define TRC_FORMAT_DRAPEAUX 19  /* unknown or inconsistent flags */
#define TRC_FORMAT_SORTE 20     /* unknown stream kind (0x05 is reserved) */
#define TRC_FORMAT_CHAMP 21     /* a field with a wrong value */
#define TRC_FORMAT_EMPREINTE 22 /* a fingerprint mismatch */
#define TRC_FORMAT_RESERVE 23   /* non-zero reserved bytes */
#define TRC_FORMAT_LIMITES 24   /* truncated or out-of-bounds structure */

#define TRC_DRAPEAU_ALIGNE 1u
#define TRC_DRAPEAU_NIVEAUX 2u
#define TRC_DRAPEAU_BRUT 4u
#define TRC_DRAPEAU_CANONIQUE 8u
#define TRC_DRAPEAU_RAPIDE 32u

#define TRC_SECTION_META 0
#define TRC_SECTION_RESIDENTS 1
#define TRC_SECTION_TABLES 2
#define TRC_SECTION_REPERTOIRE 3
#define TRC_SECTION_TRONCONS 4

#define TRC_SORTE_MEDIANES 0x01
#define TRC_SORTE_BIAIS 0x02
#define TRC_SORTE_DELTA 0x03
#define TRC_SORTE_CODES_CTX 0x04
#define TRC_SORTE_CODES_BRUTS 0x06
#define TRC_SORTE_ECHELLES_BRUTES 0x07
#define TRC_SORTE_BASE_CTX 0x10
#define TRC_SORTE_COMPL_CTX 0x11
#define TRC_SORTE_CENTRES 0x12
#define TRC_CONTEXTE_AUCUN 0xFF

typedef struct {
    uint64_t decalage;
    uint64_t longueur;
} trc_section;

/* Entete (lib.rs:250-272), read: the 4 096 on-disk bytes minus magic, alignment, header size and
 * fingerprint, which the reader checks. */
typedef struct {
    uint16_t version_majeure;
    uint16_t version_mineure;
    uint32_t drapeaux;
    uint64_t taille_fichier;
    uint8_t sha256_source[32];
    uint64_t taille_source;
    uint16_t couches;
    uint16_t experts;
    uint16_t k;
    uint16_t matrices;
    uint32_t lignes[4];
    uint32_t colonnes[4];
    uint32_t poids_par_bloc;  /* 32 */
    uint32_t octets_par_bloc; /* 17 */
    uint8_t type_ggml;        /* 39 (MXFP4) */
    uint8_t niveaux;
    uint8_t classes_echelle;
    uint8_t reserve0;
    uint8_t partition[8];
    uint32_t reserve1;
    trc_section sections[8];
} trc_entete_fichier;

/* EntreeRepertoire (lib.rs:444-500): exactly the 64 on-disk bytes. */
typedef struct {
    uint64_t decalage;
    uint32_t longueur[2];
    uint32_t utiles[2];
    uint64_t empreinte_origine;
    uint64_t empreinte_niveau[2];
    uint16_t couche;
    uint16_t expert;
    uint32_t reserve;
    uint64_t empreinte_canonique; /* v1.2 CANONIQUE files; 0 otherwise */
} trc_entree_repertoire;

/* TenseurResident (lib.rs:683-693): exactly the 128 on-disk bytes (name NUL-padded, not always
 * NUL-terminated: 64 bytes is a valid length). */
typedef struct {
    char nom[64];
    uint32_t type_ggml;
    uint32_t n_dims;
    uint64_t ne[4];
    uint64_t decalage; /* from the start of the data zone, multiple of 256 */
    uint64_t octets;
    uint64_t empreinte;
} trc_resident;

/* Table (lib.rs:518-560): the 8-byte record header, then the payload (type 1: 16 u16 frequencies,
 * 2: 256 u16 frequencies, 3: 4 f32 centres). */
typedef struct {
    uint16_t couche;
    uint8_t matrice;
    uint8_t sorte;
    uint8_t contexte;
    uint8_t type_charge;
    uint16_t reserve;
    union {
        uint16_t frequences[256];
        float centres[4];
    } charge;
} trc_table;

/* A GGUF v3 key/value pair of MÉTA (PaireMeta, meta.rs:21-30). Offsets count from the first pair
 * (byte 8 of trc_fichier_meta()'s bytes). */
typedef struct {
    uint64_t debut;     /* extent of the whole pair */
    uint64_t fin;
    uint64_t cle;       /* key bytes (UTF-8, not NUL-terminated) */
    uint64_t lg_cle;
    uint32_t type;      /* GGUF value type 0..12 */
    uint32_t type_elem; /* type 9: element type */
    uint64_t n;         /* type 9: element count; type 8: string length */
    uint64_t chaine;    /* type 8: offset of the string bytes */
    uint64_t u;         /* types 0, 2, 4, 10 and 7 (bool) */
    int64_t i;          /* types 1, 3, 5, 11 */
    double f;           /* types 6, 12 */
} trc_paire_meta;

/* DescFlux (lib.rs:780-787): exactly the 16 on-disk bytes of a stream descriptor. */
typedef struct {
    uint8_t sorte;
    uint8_t matrice;
    uint8_t contexte;
    uint8_t reserve;
    uint32_t decalage;
    uint32_t longueur;
    uint32_t produits;
} trc_desc_flux;

/* Partie (lib.rs:790-799): the part header; its descriptors are the trc_desc_flux at byte 64. */
typedef struct {
    uint16_t couche;
    uint16_t expert;
    uint8_t niveau;
    uint8_t n_matrices;
    uint16_t n_flux;
    uint32_t utiles;
} trc_partie_info;

/* empreinte64 (lib.rs:111-114): the first 8 bytes of SHA-256, little-endian. */
uint64_t trc_empreinte64(const void* octets, uint64_t n);
void trc_sha256(const void* octets, uint64_t n, uint8_t sortie[32]);
/* empreinte64 of an expert (ARCHITECTURE.md §4.12): 17-byte blocks of j = 0, 1, 2 in beta order,
 * then the f32 biases of j = 0, 1, 2. */
uint64_t trc_empreinte_expert(const uint8_t* const* blocs17, const float* const* biais, const trc_dims_expert* dims);
/* empreinte_emplacement (trc-ordo/src/lib.rs:238-262): the same from a decoded SoA slot; on a
 * CANONIQUE file it equals the directory's empreinte_canonique. */
uint64_t trc_empreinte_emplacement(const uint8_t* emplacement, const trc_dims_expert* dims);
/* lire_partie (lib.rs:813-866): structure checks of one part. */
int trc_partie_lire(const uint8_t* octets, uint64_t n, trc_partie_info* info);

/* Fichier::ouvrir (lib.rs:957-1090): header, size, sections, MÉTA, resident table, TABLES and
 * RÉPERTOIRE read and checked; parts and resident data are not read. */
typedef struct trc_fichier trc_fichier;
int trc_fichier_ouvrir(const char* chemin, trc_fichier** fichier);
void trc_fichier_fermer(trc_fichier* f);
const trc_entete_fichier* trc_fichier_entete(const trc_fichier* f);
/* Fichier::meta (lib.rs:1099-1101): u64 n then the pairs, fingerprint excluded. */
uint64_t trc_fichier_meta(const trc_fichier* f, const uint8_t** octets);
uint64_t trc_fichier_n_paires(const trc_fichier* f);
const trc_paire_meta* trc_fichier_paires(const trc_fichier* f);
/* Fichier::paire (lib.rs:1107-1109): index of the first pair with this key, -1 if none. */
int64_t trc_fichier_chercher_paire(const trc_fichier* f, const char* cle);
uint32_t trc_fichier_n_residents(const trc_fichier* f);
const trc_resident* trc_fichier_residents(const trc_fichier* f);
/* Fichier::debut_donnees_residentes (lib.rs:1114-1116): absolute offset of the data zone. */
uint64_t trc_fichier_debut_donnees(const trc_fichier* f);
/* Fichier::toutes_tables (lib.rs:1127-1129): sorted by (couche, matrice, sorte, contexte). */
uint32_t trc_fichier_n_tables(const trc_fichier* f);
const trc_table* trc_fichier_tables(const trc_fichier* f);
/* Fichier::table (lib.rs:1123-1125): NULL if absent. */
const trc_table* trc_fichier_table(const trc_fichier* f, uint16_t couche, uint8_t matrice, uint8_t sorte,
                                   uint8_t contexte);
/* luts_couche (trc-ordo/src/lib.rs:265-273): u16[3][4][256] = DELTA ctx 0, CODES_CTX ctx 0..2 of
 * each matrix, the input of trc_luts_couche. */
int trc_fichier_freqs_couche(const trc_fichier* f, uint16_t couche, uint16_t* freqs);
/* Fichier::repertoire / entree (lib.rs:1130-1137): couches x experts entries, (couche, expert) order. */
const trc_entree_repertoire* trc_fichier_repertoire(const trc_fichier* f);
const trc_entree_repertoire* trc_fichier_entree(const trc_fichier* f, uint16_t couche, uint16_t expert);
/* Fichier::octets_lus_a_l_ouverture (lib.rs:1138-1140) */
uint64_t trc_fichier_octets_lus(const trc_fichier* f);
/* Reads [decalage, decalage + octets) with pread (thread-safe). */
int trc_fichier_lire(const trc_fichier* f, uint64_t decalage, uint64_t octets, void* dst);
/* Levels 0 .. niveaux-1 of (couche, expert) in one read (longueur_jusqua, lib.rs:497-500); with
 * verifier != 0 each level is checked as trc-codec's verifier_partie and reconstruire do
 * (trc-codec/src/lib.rs:264-297): fingerprint of the useful bytes, structure, identity. */
int trc_fichier_lire_partie(const trc_fichier* f, uint16_t couche, uint16_t expert, uint32_t niveaux, void* dst,
                            uint64_t cap, int verifier, uint64_t* octets);
int trc_fichier_verifier_partie(const trc_fichier* f, uint16_t couche, uint16_t expert, uint32_t niveau,
                                const uint8_t* octets, uint64_t n);

/* Ecrivain (lib.rs:1149-1239), section by section: MÉTA, RÉSIDENTS, TABLES, then TRONÇONS
 * (directory reserved), one call per expert, terminer (directory, header). TABLES may instead come
 * after the last part, for an encoder that learns its tables layer by layer. */
typedef struct trc_ecrivain trc_ecrivain;
trc_ecrivain* trc_ecrivain_creer(const char* chemin);
void trc_ecrivain_abandonner(trc_ecrivain* w);
/* serialiser_meta (lib.rs:915-926): `paires` are n serialised GGUF v3 pairs (additions included). */
int trc_ecrivain_meta(trc_ecrivain* w, const uint8_t* paires, uint64_t octets, uint64_t n_paires);
/* disposer_residents + serialiser_table_residents (lib.rs:696-735): fills decalage and empreinte. */
int trc_ecrivain_residents(trc_ecrivain* w, trc_resident* residents, const uint8_t* const* donnees, uint32_t n);
/* serialiser_tables (lib.rs:563-583), records in the given order (the reader sorts them). */
int trc_ecrivain_tables(trc_ecrivain* w, const trc_table* tables, uint32_t n);
int trc_ecrivain_troncons(trc_ecrivain* w, uint16_t couches, uint16_t experts);
/* One expert: level 0 (level 1 after it, or NULL), each checked, written to its useful bytes and
 * padded to 4 096; the directory entry is returned in `ecrite` (may be NULL). */
int trc_ecrivain_partie(trc_ecrivain* w, uint16_t couche, uint16_t expert, const uint8_t* niveau0, uint64_t octets0,
                        const uint8_t* niveau1, uint64_t octets1, uint64_t empreinte_origine,
                        uint64_t empreinte_canonique, trc_entree_repertoire* ecrite);
/* Ecrivain::terminer (lib.rs:1227-1239): sections, size and fingerprint are filled in; frees w. */
int trc_ecrivain_terminer(trc_ecrivain* w, const trc_entete_fichier* entete, uint64_t* taille);

/* ----------------------------------------------- the expert slot cache (host only; trc-cache)
 *
 * Replaces moteur/crates/trc-cache (lib.rs:1-321, politiques.rs, trace.rs): a two-stage cache —
 * VRAM slots of decoded experts, warm-RAM entries of coded parts — with LRU, FIFO or Belady
 * replacement, and the simulator that replays a routing trace through the same code. Ids are
 * (couche << 16) | expert. */

#define TRC_POLITIQUE_LRU 0
#define TRC_POLITIQUE_BELADY 1 /* offline optimum: needs the trace of the future */
#define TRC_POLITIQUE_FIFO 2   /* LRU whose hits do not refresh */

#define TRC_CACHE_LIBRE 0
#define TRC_CACHE_EN_VOL 1  /* being decoded: never evicted */
#define TRC_CACHE_PRESENT 2

#define TRC_DECISION_SUCCES 0       /* the expert is (or will be, if in flight) in `emplacement` */
#define TRC_DECISION_DEFAUT_RAM 1   /* VRAM miss; the coded part is in warm entry `tiede` */
#define TRC_DECISION_DEFAUT_DISQUE 2 /* read the part (into `tiede` if >= 0), copy, decode */

/* ErreurTrace (trace.rs:140-152) */
#define TRC_TRACE_LIGNE 32
#define TRC_TRACE_HORS_BORNES 33
#define TRC_TRACE_VIDE 34

/* Decision (lib.rs:74-84) */
typedef struct {
    uint32_t sorte;
    uint32_t emplacement;
    int32_t tiede; /* -1: none */
    uint32_t reserve;
} trc_decision;

/* Compteurs (lib.rs:87-102), plus the RAM stage's evictions */
typedef struct {
    uint64_t succes_vram;
    uint64_t succes_ram;
    uint64_t defauts_disque;
    uint64_t octets_disque;
    uint64_t octets_copies;
    uint64_t evictions;
    uint64_t evictions_ram;
} trc_compteurs_cache;

typedef struct trc_trace trc_trace;
/* Trace::depuis_texte (trace.rs:51-130): one token per line, layers split by '|', experts by
 * blanks, '#' comments, optional "E=<n>". */
int trc_trace_depuis_texte(const char* texte, uint64_t n, trc_trace** trace);
/* choix[(t * couches + l) * k + i] */
int trc_trace_creer(uint16_t experts, uint16_t couches, uint16_t k, uint32_t jetons, const uint16_t* choix,
                    trc_trace** trace);
void trc_trace_dimensions(const trc_trace* t, uint32_t dims[4]); /* experts, couches, k, jetons */
const uint16_t* trc_trace_groupe(const trc_trace* t, uint32_t jeton, uint32_t couche);
void trc_trace_liberer(trc_trace* t);

typedef struct trc_cache trc_cache;
/* Cache::nouveau (lib.rs:111-128); `avenir` only for Belady. */
int trc_cache_creer(uint32_t emplacements, uint32_t tiedes, int politique_vram, int politique_ram,
                    const trc_trace* avenir, trc_cache** cache);
void trc_cache_detruire(trc_cache* c);
/* Cache::fixer_tailles (lib.rs:131-133): bytes read for each (couche, expert). */
int trc_cache_fixer_tailles(trc_cache* c, uint16_t couches, uint16_t experts, const uint64_t* tailles);
/* Cache::demander (lib.rs:139-180): pins the layer's experts, one decision each, in order.
 * TRC_ERREUR_USAGE when a miss finds no free or evictable slot (the cache is then unusable). */
int trc_cache_demander(trc_cache* c, uint16_t couche, const uint16_t* experts, uint32_t n, uint64_t t,
                       trc_decision* decisions);
/* Cache::pret (lib.rs:233-239): the slot's decode is done (EN_VOL -> PRESENT). */
int trc_cache_pret(trc_cache* c, uint32_t emplacement);
/* Cache::liberer (lib.rs:242-244): the layer's experts are unpinned. */
void trc_cache_liberer_couche(trc_cache* c, uint16_t couche);
trc_compteurs_cache trc_cache_compteurs(const trc_cache* c);
int trc_cache_etat(const trc_cache* c, uint32_t emplacement);
int64_t trc_cache_occupant(const trc_cache* c, uint32_t emplacement);                  /* -1: free */
int64_t trc_cache_emplacement_de(const trc_cache* c, uint16_t couche, uint16_t expert); /* -1: absent */
int64_t trc_cache_tiede_de(const trc_cache* c, uint16_t couche, uint16_t expert);      /* -1: absent */
uint32_t trc_cache_epingles(const trc_cache* c, uint32_t* ids, uint32_t max);
/* Lru::ordre (politiques.rs:93-101): VRAM ids oldest first (LRU/FIFO only, else 0). */
uint32_t trc_cache_ordre_vram(const trc_cache* c, uint32_t* ids, uint32_t max);
/* rejouer / rejouer_dans (lib.rs:282-309): the simulator. */
int trc_cache_rejouer(const trc_trace* t, uint32_t emplacements, uint32_t tiedes, int politique_vram,
                      int politique_ram, trc_compteurs_cache* compteurs);
int trc_cache_rejouer_dans(trc_cache* c, const trc_trace* t, trc_compteurs_cache* compteurs);

/* ------------------------------------------ the streaming scheduler (host over HIP; trc-ordo)
 *
 * The expert path of Moteur::pas (moteur/crates/trc-ordo/src/lib.rs:1054-1280) as a native
 * engine over an opened .trc file: per layer, router + top-k into a mapped mailbox, one wait on
 * the router's event, the cache's decisions, disk misses read at once by reader threads (pread)
 * into pinned warm entries, each part copied on a copy stream and decoded into its VRAM slot as
 * soon as it is on the host, then the layer's expert MLPs over the decoded slots (gemv_lot gate/up,
 * swiglu_oai, gemv_lot down) and the ordered combine (trc-modele/src/lib.rs:533-553). The engine
 * owns its device slots, arrival buffers, pinned entries, mailbox and copy stream (it allocates at
 * creation); the compute stream is the caller's `flux`. An error leaves the engine unusable. */

typedef struct {
    uint32_t emplacements; /* VRAM slots of decoded experts (at least k) */
    uint32_t tiedes;       /* pinned warm-RAM entries of coded parts (0: none) */
    int politique;         /* TRC_POLITIQUE_LRU or TRC_POLITIQUE_FIFO */
    int verifier;          /* check each part read against its directory fingerprint */
    uint32_t lecteurs;     /* reader threads (0: k) */
    int prechargement;     /* prefetch (Config::prechargement, trc-ordo/src/lib.rs:77,1104-1215): per
                            * layer l, layer l+1's router over the residual normed with l+1's
                            * post-attention norm (blk.N.post_attention_norm.weight if the file holds it,
                            * else unit weights; eps 1e-5) predicts its top-k; the predicted parts that
                            * are neither in VRAM nor in warm RAM are read into pinned prefetch buffers
                            * behind layer l's own reads, and a disk miss of layer l+1 without a warm
                            * entry takes its bytes from there */
    int avec_biais_cache;  /* Config::biais_cache is Some (lib.rs:110-118): the router chooses on
                            * logit + biais_cache for the layer's experts already in a VRAM slot just
                            * before the layer's cache request (routeur_topk_biais); the mixing
                            * weights stay the unbiased softmax. Refused with prechargement */
    float biais_cache;     /* beta, in raw logit units (finite) */
} trc_config_ordo;

/* CompteursMoteur (trc-ordo/src/lib.rs:586-594), the expert path's share */
typedef struct {
    uint64_t jetons;
    uint64_t lectures;
    uint64_t octets_lus;
    uint64_t octets_copies;
    uint64_t decodages;
    double us_attente_routeur; /* host time waiting for the router's event */
    double us_lectures;        /* host time from submitting the reads to the last part sent */
    double us_emission;        /* host time issuing the router and the layer's MLPs */
    uint64_t pf_emis;          /* prefetch reads issued (counted in lectures and octets_lus too) */
    uint64_t pf_utiles;        /* disk misses served from a prefetch buffer (no read of their own) */
    uint64_t pf_octets;        /* bytes of the prefetch reads */
} trc_stats_ordo;

typedef struct trc_ordo trc_ordo;
/* Moteur::nouveau (lib.rs:376-560), the expert path: slots, LUTs and routers of every layer. */
int trc_ordo_creer(const trc_fichier* f, const trc_config_ordo* cfg, trc_ordo** ordo);
/* One token through every layer's MoE part: residu += combine of the k experts chosen from x. */
int trc_ordo_jeton(trc_ordo* o, trc_vue x, trc_vue residu, void* flux);
/* Waits for flux and copies out the control words (all zero on a good run). */
int trc_ordo_controle(trc_ordo* o, uint32_t mots[4], void* flux);
trc_compteurs_cache trc_ordo_compteurs(const trc_ordo* o);
trc_stats_ordo trc_ordo_stats(const trc_ordo* o);
/* The routing the engine saw, jetons x couches x k ids (Moteur::texte_trace, lib.rs:633-649). */
uint64_t trc_ordo_trace(const trc_ordo* o, uint16_t* choix, uint64_t max);
/* The VRAM slot of a present expert (for the witness: trc_empreinte_emplacement). */
int trc_ordo_emplacement(const trc_ordo* o, uint16_t couche, uint16_t expert, trc_vue* vue);
/* The witness (trc-ordo/src/lib.rs:238-262): waits for flux, copies a present expert's slot to the
 * host and returns its empreinte64 (to compare with the directory's canonical fingerprint). */
int trc_ordo_temoin(const trc_ordo* o, uint16_t couche, uint16_t expert, void* flux, uint64_t* empreinte);
void trc_ordo_detruire(trc_ordo* o);

/* -------------------------- the streamed MoE layer on the fused path (host over HIP; trc-ordo)
 *
 * The expert part of Moteur::pas with every coded part in RAM (trc-ordo/src/lib.rs:1054-1128,
 * 1328-1370) on the fused kernels, without slots: per layer the router (gemv_f32 + routeur_topk)
 * writes the k indices into a mapped mailbox, the host waits once and reads them, the k parts are
 * copied from pinned host memory on the engine's copy stream, each expert's trc_expert_fusionne
 * starts on its copy's event, then trc_combiner. Two sets of k arrival buffers alternate between
 * consecutive layers. Residuals equal the resident step's (trc_couche_moe_fusionnee) bit for bit. */
typedef struct {
    const void* parties;       /* pinned host memory holding the layer's level-0 parts */
    const uint64_t* decalages; /* host u64[experts]: byte offset of expert e's part (16-byte aligned) */
    const uint64_t* tailles;   /* host u64[experts]: its length */
    trc_vue luts;              /* device u32[3][4][4096]: the layer's LUTs */
    trc_vue routeur;           /* device f32[experts][C]: the router (gemv_f32 over the widened rows) */
} trc_couche_hote;
typedef struct {
    uint64_t couches;           /* layers run */
    uint64_t octets_copies;     /* bytes copied host -> device */
    double us_attente_routeur;  /* host time spent waiting for the routers' events */
} trc_stats_diffusion;
typedef struct trc_diffusion trc_diffusion;
/* The engine over n_couches layers (the arrays are copied; the pinned memory, LUTs and routers must
 * outlive it), arrival buffers sized for the largest part. n_delta / n_codes as for
 * trc_expert_fusionne. */
int trc_diffusion_creer(const trc_couche_hote* couches, uint32_t n_couches, uint32_t experts, uint32_t k,
                        const trc_dims_expert* dims, uint32_t n_delta, uint32_t n_codes, trc_diffusion** sortie);
/* Layer `couche` for x on the compute stream flux: residu += combine of its k experts; the chosen
 * indices are written to choisis[k] when it is not null. A layer that fails part-way (an index out
 * of range in the mailbox, a launch error) leaves the engine refusing every later call, after its
 * queued copies and launches have drained (fail-stop, as the reference engine). */
int trc_diffusion_couche(trc_diffusion* m, uint32_t couche, trc_vue x, trc_vue residu, void* flux, uint32_t* choisis);
/* Every layer in turn for one token (the same x, as trc_ordo_jeton). */
int trc_diffusion_jeton(trc_diffusion* m, trc_vue x, trc_vue residu, void* flux);
int trc_diffusion_stats(const trc_diffusion* m, trc_stats_diffusion* s);
/* Copies out the control words of the fused experts (all zero on a good run); synchronous. */
int trc_diffusion_controle(const trc_diffusion* m, uint32_t* mots);
void trc_diffusion_detruire(trc_diffusion* m);

/* ---------------------------------------- encoder front-end (host only; role of bins/trc-codeur) */

/* The seeded synthetic workload (nibble law "A", E8M0 scales in [119,125], bf16 N(0,0.02) biases).
 * One R x C matrix of 17-byte MXFP4 blocks [e, qs16] in beta order, plus R biases. */
void trc_synth_matrice(uint64_t graine, uint32_t couche, uint32_t expert, uint32_t cle, uint32_t R, uint32_t C,
                       uint8_t* blocs17, float* biais);
/* n bf16-valued N(0, sigma) floats (activations, router weights). */
void trc_synth_normale_bf16(uint64_t graine, uint32_t cle1, uint32_t cle2, uint32_t n, float sigma, float* out);
/* Synthetic expert: gate_up generated as one (2R) x C interleaved matrix, de-interleaved into
 * j = 0 (gate, even rows) and j = 1 (up, odd rows); down is j = 2. */
int trc_synth_expert(uint64_t graine, uint32_t couche, uint32_t expert, const trc_dims_expert* dims,
                     uint8_t* const* blocs17, float* const* biais);
/* ComptesMatrice + tables() (moteur/crates/trc-codec/src/lib.rs:378-413): the 4 x 256 frequencies
 * (DELTA, CODES_CTX kappa = 0, 1, 2) of one (layer, matrix) from its experts' blocks. */
int trc_codeur_tables(const uint8_t* const* blocs17, uint32_t n_experts, uint32_t R, uint32_t B, int canonique,
                      uint16_t* freqs4);
/* coder_matrice_v10 x 3 + assembler_partie (lib.rs:417-428, trc-format/src/lib.rs:879-910):
 * a level-0 part; N_delta / N_codes macro-steps per tile. Returns the part length (0 on error). */
uint64_t trc_codeur_partie(uint16_t couche, uint16_t expert, const trc_dims_expert* dims,
                           const uint8_t* const* blocs17, const float* const* biais, const uint16_t* const* freqs4,
                           int canonique, uint32_t N_delta, uint32_t N_codes, uint8_t* out, uint64_t cap,
                           uint32_t* utiles);
/* The same with the tile lengths of each matrix j = 0, 1, 2 (N_delta[j], N_codes[j]; the format
 * stores N per stream, decisions/ARCHITECTURE.md:581, and the reference decoders honour it,
 * commun.cuh:149-157). No counterpart in the reference encoder, which always writes 256. */
uint64_t trc_codeur_partie_n(uint16_t couche, uint16_t expert, const trc_dims_expert* dims,
                             const uint8_t* const* blocs17, const float* const* biais, const uint16_t* const* freqs4,
                             int canonique, const uint32_t* N_delta, const uint32_t* N_codes, uint8_t* out,
                             uint64_t cap, uint32_t* utiles);
/* A whole synthetic layer (tables from all its experts, v1.2 parts), built on n_fils threads. */
typedef struct trc_couche_synth trc_couche_synth;
trc_couche_synth* trc_synth_couche(uint64_t graine, uint32_t couche, uint32_t n_experts, const trc_dims_expert* dims,
                                   uint32_t N_delta, uint32_t N_codes, uint32_t n_fils);
/* The same with per-matrix tile lengths (N_delta[3], N_codes[3]). */
trc_couche_synth* trc_synth_couche_n(uint64_t graine, uint32_t couche, uint32_t n_experts,
                                     const trc_dims_expert* dims, const uint32_t* N_delta, const uint32_t* N_codes,
                                     uint32_t n_fils);
uint64_t trc_synth_couche_taille(const trc_couche_synth* c, uint32_t expert);
uint32_t trc_synth_couche_utiles(const trc_couche_synth* c, uint32_t expert);
const uint8_t* trc_synth_couche_partie(const trc_couche_synth* c, uint32_t expert);
const uint16_t* trc_synth_couche_freqs(const trc_couche_synth* c); /* [3][4][256] */
/* empreinte64 of expert e as generated (canonique = 0) or with its nibbles 8 set to 0 (1). */
uint64_t trc_synth_couche_empreinte(const trc_couche_synth* c, uint32_t expert, int canonique);
void trc_synth_couche_liberer(trc_couche_synth* c);

/* FluxAEcrire (trc-format/src/lib.rs:869-876) */
typedef struct {
    uint8_t sorte;
    uint8_t matrice;
    uint8_t contexte;
    uint8_t reserve;
    uint32_t produits;
    const uint8_t* octets;
    uint64_t longueur;
} trc_flux_a_ecrire;
/* assembler_partie (trc-format/src/lib.rs:879-910): the part (length a multiple of 4 096) into
 * `out` when cap suffices; returns its length, 0 on error. */
uint64_t trc_assembler_partie(uint16_t couche, uint16_t expert, uint8_t niveau, uint8_t n_matrices,
                              const trc_flux_a_ecrire* flux, uint32_t n, uint8_t* out, uint64_t cap,
                              uint32_t* utiles);
/* A whole synthetic model as a v1.2 CANONIQUE .trc file (role of bins/trc-codeur/src/coder.rs:114-
 * 390 on a GGUF): layer c's experts are those of trc_synth_couche(graine, c, ...), its router
 * "blk.<c>.ffn_gate_inp.weight" (bf16, experts x colonnes[0]) the bf16 N(0, 0.02) rows
 * trc_synth_normale_bf16(graine + c, 3, e, ...), MÉTA holds gpt-oss-style hyper-parameters, TABLES
 * follow the parts. Layers are generated one at a time on n_fils threads. */
int trc_synth_fichier(const char* chemin, uint64_t graine, uint16_t couches, uint16_t experts, uint16_t k,
                      const trc_dims_expert* dims, uint32_t N_delta, uint32_t N_codes, uint32_t n_fils,
                      uint64_t* taille);

#ifdef __cplusplus
}
#endif
#endif
