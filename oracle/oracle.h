/*
 * oracle.h — CPU restatement of the reference (troncons) algorithms on the expert hot path.
 *
 * THIS IS TEST INFRASTRUCTURE, NOT PRODUCT CODE. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it, and only as the checker / CPU baseline. The product
 * (troncons_amd/) never links or calls it.
 *
 * Every function restates a reference function from its text (cited file:line, paths relative to
 * the reference tree). The reference is Rust + CUDA and cannot be compiled in this image (no Rust
 * toolchain, no nvcc), so nothing here is a build of the reference itself.
 *
 * Pinning (what checks each function, beyond round trips) is listed next to each declaration:
 *   KAT   = known answer from the reference's own tests,
 *   MATH  = closed form / hand-derived value / brute force on tiny inputs (tests/test_oracle_*.py).
 * A function marked "parity unpinned" has no such check.
 */
#ifndef TRC_ORACLE_H
#define TRC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* rANS constants — moteur/crates/trc-codec/src/rans.rs:25-38 */
#define ORC_M 4096u
#define ORC_L 65536u
#define ORC_VOIES 32u
#define ORC_OCTETS_PAR_MACRO 128u
#define ORC_ENTETE_FLUX 16u

/* ------------------------------------------------------------------------------------- tables */

/* TableRans::depuis_comptes (rans.rs:83-127). geometrie 1 (256 symbols) or 2 (16 symbols).
 * freq_out receives n_symbols u16 summing to 4096.  Pinned: KAT (tests/rans.rs:253-254 all-zero
 * counts), MATH (hand-derived tie-break cases for both geometries). */
void orc_table_depuis_comptes(const uint64_t* comptes, int geometrie, uint16_t* freq_out);

/* TableRans::construire (rans.rs:146-166): cumulative table and 4096-entry LUT.
 * Returns 0, or -1 if the frequencies do not sum to 4096 or one exceeds 4096
 * (TableRans::depuis_frequences, rans.rs:131-144).  Pinned: KAT abi.rs:385-406. */
int orc_lut(const uint16_t* freq, int geometrie, uint32_t* cumul_out /* may be NULL */, uint32_t* lut_out);

/* luts_couche (abi.rs:210-221): u32[3][4][4096]; freqs[j*4+t] = 256 frequencies or NULL
 * (absent table = zero LUT). Returns 0 or -1. */
int orc_luts_couche(const uint16_t* const* freqs, uint32_t* luts_out);

/* ------------------------------------------------------------------------------------- stream */

typedef struct {
    uint32_t P;        /* bytes produced (multiple of 128) */
    uint32_t N;        /* macro-steps per tile */
    uint32_t geometrie;
    uint32_t T;        /* tiles */
    uint32_t W;        /* 16-bit words */
    const uint8_t* debuts; /* T x u32 LE */
    const uint8_t* etats;  /* 32T x u32 LE */
    const uint8_t* mots;   /* W x u16 LE */
} orc_flux;

/* FluxRans::lire (rans.rs:231-280): parse + all header checks. 0 or -1. */
int orc_flux_lire(const uint8_t* b, size_t len, orc_flux* out);

/* Bilan (rans.rs:368-382) */
typedef struct {
    uint64_t voies_hors_l;
    uint64_t tuiles_mots_faux;
    int64_t premiere_tuile; /* -1 if none */
} orc_bilan;

/* coder_avec (rans.rs:296-334) + FluxRans::serialiser (rans.rs:208-227), with N macro-steps per
 * tile as a parameter (the reference encoder fixes N = 256; the format stores N per stream,
 * ARCHITECTURE.md:581). source: P bytes, P % 128 == 0.
 * Context of symbol n: geometrie 1 -> kappa[n/16] (0 beyond n_kappa) if kappa != NULL, else 0
 * (coder_par_voie rans.rs:359-362 / DELTA lib.rs:419); geometrie 2 -> table 0.
 * freqs: ntables x n_symbols u16. Returns serialized length (written to out if out != NULL and
 * cap is large enough), or 0 on error (symbol absent from its table, bad sizes). */
size_t orc_coder(const uint8_t* source, size_t P, int geometrie, const uint8_t* kappa, size_t n_kappa,
                 const uint16_t* freqs, int ntables, uint32_t N, uint8_t* out, size_t cap);

/* decoder_avec (rans.rs:388-451) over a parsed stream; contexts as in orc_coder; luts: ntables x
 * 4096 u32. out receives P bytes (geometrie 2: P bytes of packed nibbles). 0 or -1 (context
 * without table). */
int orc_decoder(const orc_flux* f, const uint8_t* kappa, size_t n_kappa, const uint32_t* luts, int ntables,
                uint8_t* out, orc_bilan* bilan);

/* ------------------------------------------------------------------------------ matrix codec */

/* classe_echelle (lib.rs:48-55) */
uint8_t orc_classe_echelle(uint8_t delta);

/* canoniser_octet (trc-format/src/lib.rs:74-83) */
uint8_t orc_canoniser_octet(uint8_t o);

/* preparer_matrice_avec (lib.rs:348-373). blocs: R*B blocks of 17 bytes [e, qs16].
 * medianes: R; delta: padded to ceil(R*B/128)*128; qs: padded to ceil(16*R*B/128)*128. */
void orc_preparer_matrice(const uint8_t* blocs, uint32_t R, uint32_t B, int canonique, uint8_t* medianes,
                          uint8_t* delta, uint8_t* qs);

/* ComptesMatrice::ajouter (lib.rs:390-398): delta_c[256], codes_c[3][256] += counts. */
void orc_comptes_ajouter(const uint8_t* delta, size_t n_delta, const uint8_t* qs, size_t n_qs, uint64_t* delta_c,
                         uint64_t* codes_c);

/* Part assembly / reading — assembler_partie (trc-format/src/lib.rs:879-910), lire_partie
 * (:813-877). A stream descriptor: */
typedef struct {
    uint8_t sorte, matrice, contexte;
    uint32_t decalage, longueur, produits;
} orc_desc_flux;

/* Returns total length (multiple of 4096) and *utiles; writes to out if cap suffices. */
size_t orc_assembler_partie(uint16_t couche, uint16_t expert, uint8_t niveau, uint8_t n_matrices, int n_flux,
                            const uint8_t* sortes, const uint8_t* matrices, const uint8_t* contextes,
                            const uint32_t* produits, const uint8_t* const* octets, const uint32_t* longueurs,
                            uint8_t* out, size_t cap, uint32_t* utiles);

typedef struct {
    uint16_t couche, expert;
    uint8_t niveau, n_matrices;
    uint32_t n_flux, utiles;
    orc_desc_flux flux[64];
} orc_partie;

/* lire_partie: 0 or -1 (every refusal of the reference reader). */
int orc_lire_partie(const uint8_t* octets, size_t len, orc_partie* p);

/* Encode one matrix v1.0/v1.2 into its four streams and append them to a part under
 * construction: coder_matrice_v10 (lib.rs:417-428). Convenience for tests: see orc_coder_expert. */

/* Full expert encode: 3 matrices (R[j] x C[j]), blocks17[j], biases f32 bytes bias[j] (4R each),
 * given per-matrix tables freqs[j] = {delta[256], codes0[256], codes1[256], codes2[256]}.
 * N_delta / N_codes: macro-steps per tile. canonique: v1.2 folding. Returns part length. */
size_t orc_coder_expert(uint16_t couche, uint16_t expert, int n_matrices, const uint32_t* R, const uint32_t* C,
                        const uint8_t* const* blocs17, const uint8_t* const* biais, const uint16_t* const* freqs,
                        int canonique, uint32_t N_delta, uint32_t N_codes, uint8_t* out, size_t cap,
                        uint32_t* utiles);

/* Tables of one (layer, matrix) from the blocks of several experts: ComptesMatrice + tables()
 * (lib.rs:378-413). blocs17: n_experts pointers. freqs_out: 4 x 256 (delta, codes k=0..2). */
void orc_tables_matrice(const uint8_t* const* blocs17, int n_experts, uint32_t R, uint32_t B, int canonique,
                        uint16_t* freqs_out);

/* Reconstruction of one matrix from a level-0 part: decoder_matrice_v10 (lib.rs:190-218).
 * codes: 16*R*B, echelles: R*B, biais: 4R bytes. bd/bc: bilans of DELTA and CODES_CTX.
 * Returns 0 or -1 (format error). luts: the matrix's 4 LUTs u32[4][4096] ([0] DELTA). */
int orc_decoder_matrice(const uint8_t* partie, size_t len, uint8_t j, uint32_t R, uint32_t B,
                        const uint32_t* luts4, uint8_t* codes, uint8_t* echelles, uint8_t* biais,
                        orc_bilan* bd, orc_bilan* bc);

/* SoA slot layout (abi.rs:69-122, commun.cuh:49-92). */
typedef struct {
    uint64_t base, echelles, biais, pas;
} orc_disposition;
orc_disposition orc_disposition_matrice(uint32_t lignes, uint32_t colonnes);
uint64_t orc_taille_emplacement(const uint32_t* lignes, const uint32_t* colonnes);
orc_disposition orc_disposition_j(const uint32_t* lignes, const uint32_t* colonnes, int j);

/* Decode a 3-matrix expert part into a slot (what decoder_expert must produce). ctl[4] gets
 * {lanes off L, format errors, tiles with wrong word count, 0}. luts: u32[3][4][4096].
 * Returns 0 or -1. */
int orc_decoder_expert(const uint8_t* partie, size_t len, const uint32_t* luts, const uint32_t* lignes,
                       const uint32_t* colonnes, uint8_t* emplacement, uint32_t* ctl);

/* ------------------------------------------------------------------------------- arithmetic */

/* 2^(e-128) as f32 (gemv.cuh:26-29) and the doubled E2M1 value (gemv.cuh:33-36). */
float orc_echelle_e8m0(uint32_t e);
float orc_valeur_e2m1x2(uint32_t c);

/* gemv_mxfp4 on one slot matrix, in the reference's exact f32 operation order (gemv.cuh:60-126):
 * lane l takes blocks l, l+32, ...; 32 fmaf per block in (word, byte, low nibble, high nibble)
 * order; acc = fmaf(scale, dot, acc); 32-lane butterfly; y = sum + bias. */
void orc_gemv_mxfp4(const uint8_t* matrice, const float* x, float* y, uint32_t R, uint32_t C);

/* f64 reference y = W x + b over the same slot matrix (banc_k.cu:1047-1072, carte.rs:374-406). */
void orc_gemv_mxfp4_f64(const uint8_t* matrice, const float* x, double* y, uint32_t R, uint32_t C);

/* gemv_f32 (passe.cuh:104-130): y = W x (+ b), W row-major f32 R x C, reference order. */
void orc_gemv_f32(const float* W, const float* x, const float* biais, float* y, uint32_t R, uint32_t C);

/* swiglu_oai (passe.cuh:598-605, trc-reference ops.rs:133-140), f64 then one rounding. */
void orc_swiglu_oai(const float* g, const float* u, float* y, uint32_t n);

/* combiner (passe.cuh:611-622): residu[i] += ((w0 s0 + w1 s1) + w2 s2) + ..., no FMA. */
void orc_combiner(float* residu, const float* sorties, uint32_t pas, const float* poids, uint32_t n, uint32_t d);

/* routeur_topk (passe.cuh:455-514, ops.rs:121-131): top-k by (value desc, index asc), softmax of
 * the k in f64 (m = first), rounded to f32. */
void orc_routeur_topk(const float* logits, uint32_t E, uint32_t k, uint32_t* indices, float* poids);
/* routeur_topk_biais (passe.cuh:516-580). Pinned by: zero bias gives orc_routeur_topk bit for bit;
 * a sort-based restatement (the reference's host version, tests/passe.rs:328-337) on tie-forcing
 * draws; a hand case whose weights are a closed-form softmax. */
void orc_routeur_topk_biais(const float* logits, const float* biais, uint32_t E, uint32_t k, uint32_t* indices,
                            float* poids);

/* ------------------------------------------------------------- forward pass around the experts */
/* (passe.c) The rest of a gpt-oss layer step, in each reference kernel's operation order. */

/* ParamsRope (trc-noyaux/src/abi.rs:229-251, passe.cuh:134-143): 48 bytes. */
typedef struct {
    double base, facteur, ctx_origine, beta_rapide, beta_lent;
    uint32_t dim_tete, variante;
} orc_params_rope;
/* ParamsAttention (abi.rs:253-291, passe.cuh:171-181): 32 bytes. */
typedef struct {
    uint32_t tetes, tetes_kv, dim_tete, debut, fin, anneau;
    float echelle;
    uint32_t reserve;
} orc_params_attention;

/* f16 <-> f32: f32 -> f16 rounds to nearest even (overflow to inf, subnormals kept).
 * KAT: the eight values of tests/passe.rs:146-159; MATH: numpy's float16 on every f16 and on
 * random f32 (tests/test_oracle_passe.py). */
float orc_f32_depuis_f16(uint16_t h);
uint16_t orc_f16_depuis_f32(float f);
/* gemv_q8_0 (passe.cuh:52-97): KAT integer-exact fixture of tests/passe.rs:83-118 (equal to the
 * f64 sum, bias included); MATH: f64 within 1e-6 on random data. The lane order itself is the
 * reference text's (no reference output pins it): the GPU kernel, written apart, must equal it
 * bit for bit. */
void orc_gemv_q8_0(const uint8_t* W, const float* x, const float* biais, float* y, uint32_t R, uint32_t C);
/* ligne_q8_0 (passe.cuh:627-637): KAT tests/passe.rs:127-145 (d = 2^e, exact). */
void orc_ligne_q8_0(const uint8_t* W, uint32_t ligne, uint32_t C, float* y);
/* rmsnorm (passe.cuh:235-259): MATH: the f64 closed form of ops.rs:8-18 within 1e-6
 * (tests/passe.rs:163-176). */
void orc_rmsnorm(const float* x, const float* w, float* y, uint32_t n, uint32_t lignes, float eps);
/* YaRN inv_freq (passe.cuh:145-167): KAT ramp bounds 8.0928 / 17.3981 and 8 / 18 (llama.cpp
 * variant), concentration 0.1 ln 32 + 1, variants equal outside the ramp (ops.rs:146-163). */
double orc_inv_freq_yarn(const orc_params_rope* p, uint32_t i, double* concentration, double* bas, double* haut);
/* rope_yarn (passe.cuh:261-284): KAT position 0 = times the concentration, factor 1 at position
 * 1000 = plain RoPE (tests/passe.rs:177-200); MATH: norm times concentration^2 (ops.rs:165-173). */
void orc_rope_yarn(float* q, float* k, uint32_t tetes_q, uint32_t tetes_k, uint32_t position,
                   const orc_params_rope* p);
/* ecrire_kv (passe.cuh:286-296): via orc_f16_depuis_f32; slot placement checked by the KAT. */
void orc_ecrire_kv(const float* k, const float* v, uint16_t* cache_k, uint16_t* cache_v, uint32_t dkv,
                   uint32_t case_kv);
/* attention (passe.cuh:298-373): KAT sink in the denominator (ops.rs:175-186), ring of 128 at
 * position 200 (mean 63.5) and 4096 positions (mean 1023.5) of tests/passe.rs:217-272; MATH: the
 * f64 definition of ops.rs:87-118 within 1e-5 on random heads. */
void orc_attention(const float* q, const uint16_t* cache_k, const uint16_t* cache_v, const float* puits,
                   float* sortie, const orc_params_attention* p);
/* argmax (passe.cuh:639-666): KAT tests/passe.rs:296-302 (tie -> lower index, NaN never). */
uint32_t orc_argmax(const float* v, uint32_t n);

/* ------------------------------------------------------------------------------ generators */

/* splitmix64 as in moteur/crates/trc-noyaux/tests/carte.rs:22-31 (state advanced first). */
uint64_t orc_splitmix64(uint64_t* etat);
/* xorshift64* as in moteur/crates/trc-codec/tests/rans.rs:20-27. */
uint64_t orc_xorshift64s(uint64_t* etat);

/* bf16 <-> f32 (round to nearest even; NaN kept quiet). */
uint16_t orc_bf16_depuis_f32(float f);
float orc_f32_depuis_bf16(uint16_t h);

/* The synthetic workload of this build (the benchmark configurations: MXFP4 law A, E8M0 in
 * [119, 125], bf16 N(0, 1) activations, bf16 N(0, 0.02) router):
 * orc_synth_matrice fills blocks17 (R*B x 17) and bias (R f32, bf16-valued) for a
 * (seed, layer, expert, matrix-slot) key; see synth.c for the exact draw order. */
void orc_synth_matrice(uint64_t graine, uint32_t couche, uint32_t expert, uint32_t cle, uint32_t R, uint32_t C,
                       uint8_t* blocs17, float* biais);
/* bf16 N(0, sigma) vector (values returned as f32), keyed like the matrices. */
void orc_synth_normale_bf16(uint64_t graine, uint32_t cle1, uint32_t cle2, uint32_t n, float sigma, float* out);

/* empreinte64 (trc-format/src/lib.rs:111-116): first 8 bytes of SHA-256 as LE u64. */
uint64_t orc_empreinte64(const uint8_t* octets, size_t n);

#ifdef __cplusplus
}
#endif
#endif
