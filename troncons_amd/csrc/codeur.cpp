// codeur.cpp — the encoder front-end of the hot path (the role of bins/trc-codeur for this build):
// seeded synthetic MXFP4 experts of gpt-oss shape, per-(layer, matrix) tables from counts over all
// experts of a layer, and .trc v1.2 level-0 parts (MEDIANES, BIAIS, DELTA, CODES_CTX per matrix).
//
// Host C++, multi-threaded with std::thread. The algorithms restate moteur/crates/trc-codec/src/
// rans.rs (normalisation :83-127, coder_avec :296-334, serialiser :208-227), trc-codec/src/lib.rs
// (preparer_matrice_avec :348-373, ComptesMatrice :378-413, coder_matrice_v10 :417-428) and
// trc-format/src/lib.rs (assembler_partie :879-910). Unlike the reference encoder, which always
// writes N = 256 macro-steps per tile, the tile length is a parameter (the format stores N per
// stream and every decoder honours it): short tiles are the parallelism the GPU decoder needs.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <memory>
#include <thread>
#include <vector>

#include "commun.hpp"
#include "erreurs.hpp"

namespace {

// ------------------------------------------------------------------------------- generators

struct SplitMix64 {
    uint64_t etat;
    uint64_t suivant() {
        etat += 0x9E3779B97F4A7C15ull;
        uint64_t z = etat;
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniforme53() { return double(suivant() >> 11) * 0x1.0p-53; }
};

uint64_t etat_initial(uint64_t graine, uint32_t couche, uint32_t expert, uint32_t cle) {
    const uint64_t k = (uint64_t(couche & 0xFFFFFFu) << 40) ^ (uint64_t(expert & 0xFFFFFFu) << 16) ^ uint64_t(cle & 0xFFFFu);
    return graine ^ (k * 0xD1B54A32D192ED03ull);
}

uint16_t bf16(float f) {
    uint32_t b;
    std::memcpy(&b, &f, 4);
    if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x7FFFFFu)) return uint16_t((b >> 16) | 0x40);
    return uint16_t((b + 0x7FFFu + ((b >> 16) & 1u)) >> 16);
}

float depuis_bf16(uint16_t h) {
    const uint32_t b = uint32_t(h) << 16;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

// The nibble law of the synthetic workload: symmetric, peaked, zero with a random sign (the v1.2
// fold of -0 into +0 brings p(0) to 0.20).
constexpr double LOI_A[16] = {0.10, 0.14, 0.13, 0.06, 0.035, 0.02, 0.01, 0.005,
                              0.10, 0.14, 0.13, 0.06, 0.035, 0.02, 0.01, 0.005};

struct Cdf {
    double c[16];
    Cdf() {
        double a = 0.0;
        for (int i = 0; i < 16; ++i) {
            a += LOI_A[i];
            c[i] = a;
        }
    }
    uint32_t tirer(SplitMix64& g) const {
        const double u = g.uniforme53();
        for (uint32_t i = 0; i < 15; ++i)
            if (u < c[i]) return i;
        return 15;
    }
};

void normales(SplitMix64& g, uint32_t n, float sigma, float* out) {
    for (uint32_t i = 0; i < n; i += 2) {
        const double u1 = double((g.suivant() >> 11) + 1) * 0x1.0p-53;
        const double u2 = double(g.suivant() >> 11) * 0x1.0p-53;
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double a = 6.283185307179586 * u2;
        out[i] = depuis_bf16(bf16(float(double(sigma) * (r * std::cos(a)))));
        if (i + 1 < n) out[i + 1] = depuis_bf16(bf16(float(double(sigma) * (r * std::sin(a)))));
    }
}

// One R x C matrix of 17-byte blocks [e, qs16] in beta order, and its R biases.
void synth_matrice(uint64_t graine, uint32_t couche, uint32_t expert, uint32_t cle, uint32_t R, uint32_t C,
                   uint8_t* blocs, float* biais) {
    SplitMix64 g{etat_initial(graine, couche, expert, cle)};
    static const Cdf cdf;
    const uint64_t nb = uint64_t(R) * (C / 32);
    for (uint64_t b = 0; b < nb; ++b) blocs[17 * b] = uint8_t(119 + g.suivant() % 7);
    for (uint64_t b = 0; b < nb; ++b)
        for (int i = 0; i < 16; ++i) {
            const uint32_t lo = cdf.tirer(g);
            const uint32_t hi = cdf.tirer(g);
            blocs[17 * b + 1 + i] = uint8_t(lo | (hi << 4));
        }
    if (biais) normales(g, R, 0.02f, biais);
}

// ------------------------------------------------------------------------------ rANS tables

uint8_t classe(uint8_t d) { return d < 128 ? 0 : (d == 128 ? 1 : 2); }

uint8_t canonique(uint8_t o) {
    uint8_t lo = o & 15, hi = o >> 4;
    if (lo == 8) lo = 0;
    if (hi == 8) hi = 0;
    return uint8_t(lo | (hi << 4));
}

// TableRans::depuis_comptes, geometry 1 (rans.rs:83-127).
void normaliser(const uint64_t* comptes_in, uint16_t* freq_out) {
    uint64_t c[256];
    uint64_t total = 0;
    for (int i = 0; i < 256; ++i) total += (c[i] = comptes_in[i]);
    if (total == 0) {
        c[0] = 1;
        total = 1;
    }
    int64_t f[256];
    for (int i = 0; i < 256; ++i) {
        f[i] = 0;
        if (c[i] > 0) f[i] = std::max<int64_t>(1, int64_t(std::round(double(c[i]) * 4096.0 / double(total))));
    }
    int64_t somme = 0;
    for (int i = 0; i < 256; ++i) somme += f[i];
    std::vector<int> ordre(256);
    for (int i = 0; i < 256; ++i) ordre[i] = i;
    std::stable_sort(ordre.begin(), ordre.end(), [&](int a, int b) { return f[a] > f[b]; });
    for (size_t j = 0; somme != 4096; ++j) {
        const int i = ordre[j % 256];
        if (somme > 4096 && f[i] > 1) {
            --f[i];
            --somme;
        } else if (somme < 4096 && f[i] > 0) {
            ++f[i];
            ++somme;
        }
    }
    for (int i = 0; i < 256; ++i) freq_out[i] = uint16_t(f[i]);
}

struct Table {
    uint32_t f[256];
    uint32_t c[256];
    explicit Table(const uint16_t* freq) {
        uint32_t a = 0;
        for (int s = 0; s < 256; ++s) {
            f[s] = freq[s];
            c[s] = a;
            a += freq[s];
        }
    }
};

size_t pad128(size_t n) { return (n + 127) / 128 * 128; }

// A prepared matrix: medians, padded deltas, padded (canonical) code bytes.
struct Prepa {
    std::vector<uint8_t> med, delta, qs;
};

void preparer(const uint8_t* blocs, uint32_t R, uint32_t B, bool canon, Prepa& p) {
    const size_t nb = size_t(R) * B;
    p.med.assign(R, 0);
    p.delta.assign(pad128(nb), 0);
    p.qs.assign(pad128(16 * nb), 0);
    std::vector<uint8_t> tri(B);
    for (uint32_t r = 0; r < R; ++r) {
        const uint8_t* ligne = blocs + size_t(r) * B * 17;
        for (uint32_t i = 0; i < B; ++i) tri[i] = ligne[17 * i];
        std::nth_element(tri.begin(), tri.begin() + B / 2, tri.end());
        const uint8_t med = tri[B / 2];
        p.med[r] = med;
        for (uint32_t i = 0; i < B; ++i) {
            const size_t beta = size_t(r) * B + i;
            p.delta[beta] = uint8_t(ligne[17 * i] - med + 128);
            for (int k = 0; k < 16; ++k) {
                const uint8_t o = ligne[17 * i + 1 + k];
                p.qs[16 * beta + k] = canon ? canonique(o) : o;
            }
        }
    }
}

void compter(const Prepa& p, uint64_t* delta_c, uint64_t* codes_c) {
    for (uint8_t d : p.delta) delta_c[d]++;
    const size_t n_delta = p.delta.size();
    for (size_t n = 0; n < p.qs.size(); ++n) {
        const size_t blk = n / 16;
        codes_c[256 * classe(blk < n_delta ? p.delta[blk] : 0) + p.qs[n]]++;
    }
}

// coder_avec + serialiser (rans.rs:296-334, 208-227), geometry 1, N macro-steps per tile.
// kappa: context of byte n = kappa[n/16] (0 beyond), or nullptr for a single table.
std::vector<uint8_t> coder(const std::vector<uint8_t>& src, const std::vector<uint8_t>* kappa,
                           const Table* const* tables, uint32_t N) {
    const size_t P = src.size();
    const size_t n_macro = P / 128;
    const size_t T = (n_macro + N - 1) / N;
    std::vector<uint32_t> debuts(T), etats(32 * T);
    std::vector<uint16_t> mots;
    mots.reserve(P / 2);
    std::vector<uint16_t> pile;
    pile.reserve(size_t(N) * 128);
    for (size_t t = 0; t < T; ++t) {
        const size_t m0 = t * N, nb = std::min<size_t>(N, n_macro - m0);
        uint64_t x[32];
        for (int l = 0; l < 32; ++l) x[l] = trc::L;
        pile.clear();
        for (size_t m = nb; m-- > 0;)
            for (int k = 3; k >= 0; --k)
                for (int l = 31; l >= 0; --l) {
                    const size_t n = ((m0 + m) * 32 + size_t(l)) * 4 + size_t(k);
                    int ctx = 0;
                    if (kappa) {
                        const size_t blk = n / 16;
                        ctx = blk < kappa->size() ? (*kappa)[blk] : 0;
                    }
                    const Table& tb = *tables[ctx];
                    const uint32_t s = src[n];
                    const uint64_t f = tb.f[s];
                    if (f == 0) return {};  // symbol absent from its table: caller error
                    uint64_t xv = x[l];
                    if (xv >= (f << 20)) {
                        pile.push_back(uint16_t(xv & 0xFFFF));
                        xv >>= 16;
                    }
                    x[l] = ((xv / f) << 12) + (xv % f) + tb.c[s];
                }
        debuts[t] = uint32_t(mots.size());
        for (int l = 0; l < 32; ++l) etats[32 * t + l] = uint32_t(x[l]);
        mots.insert(mots.end(), pile.rbegin(), pile.rend());
    }
    size_t len = 16 + 4 * T + 128 * T + 2 * mots.size();
    len = (len + 15) / 16 * 16;
    std::vector<uint8_t> o(len, 0);
    auto w32 = [&](size_t p, uint32_t v) { std::memcpy(&o[p], &v, 4); };
    w32(0, uint32_t(P));
    o[4] = uint8_t(N);
    o[5] = uint8_t(N >> 8);
    o[6] = 1;
    w32(8, uint32_t(T));
    w32(12, uint32_t(mots.size()));
    std::memcpy(&o[16], debuts.data(), 4 * T);
    std::memcpy(&o[16 + 4 * T], etats.data(), 128 * T);
    if (!mots.empty()) std::memcpy(&o[16 + 132 * T], mots.data(), 2 * mots.size());
    return o;
}

struct FluxEcrit {
    uint8_t sorte, matrice, contexte;
    uint32_t produits;
    std::vector<uint8_t> octets;
};

// assembler_partie (trc-format/src/lib.rs:879-910): header, descriptors, streams on 16-byte
// boundaries, zeros up to a multiple of 4 096. Magic "TRC0" for level 0, "TRC1" for level 1.
std::vector<uint8_t> assembler(uint16_t couche, uint16_t expert, uint8_t n_mat, const std::vector<FluxEcrit>& flux,
                               uint32_t& utiles, uint8_t niveau = 0) {
    size_t p = 64 + 16 * flux.size();
    std::vector<size_t> dec(flux.size());
    for (size_t i = 0; i < flux.size(); ++i) {
        p = (p + 15) / 16 * 16;
        dec[i] = p;
        p += flux[i].octets.size();
    }
    utiles = uint32_t(p);
    std::vector<uint8_t> b((p + 4095) / 4096 * 4096, 0);
    auto w16 = [&](size_t q, uint32_t v) { b[q] = uint8_t(v); b[q + 1] = uint8_t(v >> 8); };
    auto w32 = [&](size_t q, uint32_t v) { std::memcpy(&b[q], &v, 4); };
    w32(0, niveau == 0 ? trc::MAGIE_PARTIE0 : 0x31435254u);
    w16(4, couche);
    w16(6, expert);
    b[8] = niveau;
    b[9] = n_mat;
    w16(10, uint32_t(flux.size()));
    w32(12, utiles);
    for (size_t i = 0; i < flux.size(); ++i) {
        const size_t q = 64 + 16 * i;
        b[q] = flux[i].sorte;
        b[q + 1] = flux[i].matrice;
        b[q + 2] = flux[i].contexte;
        w32(q + 4, uint32_t(dec[i]));
        w32(q + 8, uint32_t(flux[i].octets.size()));
        w32(q + 12, flux[i].produits);
        if (!flux[i].octets.empty()) std::memcpy(&b[dec[i]], flux[i].octets.data(), flux[i].octets.size());
    }
    return b;
}

// coder_matrice_v10 (lib.rs:417-428) for matrix j, appended to `flux`.
bool coder_matrice(const Prepa& p, uint32_t R, const float* biais, const uint16_t* freqs4, uint8_t j,
                   uint32_t N_delta, uint32_t N_codes, std::vector<FluxEcrit>& flux) {
    const Table td(freqs4), t0(freqs4 + 256), t1(freqs4 + 512), t2(freqs4 + 768);
    const Table* tdelta[1] = {&td};
    const Table* tcodes[3] = {&t0, &t1, &t2};
    std::vector<uint8_t> kappa(p.delta.size());
    for (size_t i = 0; i < p.delta.size(); ++i) kappa[i] = classe(p.delta[i]);
    std::vector<uint8_t> fd = coder(p.delta, nullptr, tdelta, N_delta);
    std::vector<uint8_t> fc = coder(p.qs, &kappa, tcodes, N_codes);
    if (fd.empty() || fc.empty()) return false;
    std::vector<uint8_t> bi(4 * size_t(R));
    std::memcpy(bi.data(), biais, 4 * size_t(R));
    flux.push_back({trc::SORTE_MEDIANES, j, 0xFF, R, p.med});
    flux.push_back({trc::SORTE_BIAIS, j, 0xFF, 4 * R, std::move(bi)});
    flux.push_back({trc::SORTE_DELTA, j, 0, uint32_t(p.delta.size()), std::move(fd)});
    flux.push_back({trc::SORTE_CODES_CTX, j, 0xFF, uint32_t(p.qs.size()), std::move(fc)});
    return true;
}

template <typename F>
void en_parallele(uint32_t n, uint32_t n_fils, F&& f) {
    n_fils = std::max(1u, std::min(n_fils, n));
    std::atomic<uint32_t> suivant{0};
    std::vector<std::thread> fils;
    for (uint32_t k = 0; k < n_fils; ++k)
        fils.emplace_back([&] {
            for (uint32_t i; (i = suivant.fetch_add(1)) < n;) f(i);
        });
    for (auto& t : fils) t.join();
}

}  // namespace

// ==================================================================================== C-ABI

struct trc_couche_synth {
    std::vector<std::vector<uint8_t>> parties;
    std::vector<uint32_t> utiles;
    std::vector<uint64_t> empreinte_origine;    // of the generated expert
    std::vector<uint64_t> empreinte_canonique;  // of the same with every nibble 8 of qs set to 0
    uint16_t freqs[3][4][256];
};

extern "C" {

void trc_synth_matrice(uint64_t graine, uint32_t couche, uint32_t expert, uint32_t cle, uint32_t R, uint32_t C,
                       uint8_t* blocs17, float* biais) {
    synth_matrice(graine, couche, expert, cle, R, C, blocs17, biais);
}

void trc_synth_normale_bf16(uint64_t graine, uint32_t cle1, uint32_t cle2, uint32_t n, float sigma, float* out) {
    SplitMix64 g{etat_initial(graine, cle1, 0xFFFFFFu, cle2)};
    normales(g, n, sigma, out);
}

// The three matrices of synthetic expert e of a layer: gate_up is one (2R) x C matrix with
// interleaved rows (row 2i gate i, row 2i+1 up i), de-interleaved into j = 0 (gate) and j = 1
// (up); down is j = 2. blocs[j]: R_j*B_j*17 bytes, biais[j]: R_j floats.
int trc_synth_expert(uint64_t graine, uint32_t couche, uint32_t expert, const trc_dims_expert* dims,
                     uint8_t* const* blocs, float* const* biais) {
    if (dims == nullptr || blocs == nullptr || biais == nullptr) return trc::usage("pointeur nul");
    if (dims->lignes[0] != dims->lignes[1] || dims->colonnes[0] != dims->colonnes[1])
        return trc::usage("gate et up de formes differentes");
    const int r = trc_dims_verifier(dims);
    if (r != TRC_OK) return r;
    const uint32_t R = dims->lignes[0], C = dims->colonnes[0], B = C / 32;
    std::vector<uint8_t> gu(size_t(2 * R) * B * 17);
    std::vector<float> bgu(2 * R);
    synth_matrice(graine, couche, expert, 1, 2 * R, C, gu.data(), bgu.data());
    const size_t ligne = size_t(B) * 17;
    for (uint32_t i = 0; i < R; ++i) {
        std::memcpy(blocs[0] + i * ligne, gu.data() + (2 * i) * ligne, ligne);
        std::memcpy(blocs[1] + i * ligne, gu.data() + (2 * i + 1) * ligne, ligne);
        biais[0][i] = bgu[2 * i];
        biais[1][i] = bgu[2 * i + 1];
    }
    synth_matrice(graine, couche, expert, 2, dims->lignes[2], dims->colonnes[2], blocs[2], biais[2]);
    return TRC_OK;
}

// Tables of one (layer, matrix) from counts over n experts (ComptesMatrice + tables()).
int trc_codeur_tables(const uint8_t* const* blocs17, uint32_t n_experts, uint32_t R, uint32_t B, int canon,
                      uint16_t* freqs4) {
    if (blocs17 == nullptr || freqs4 == nullptr || R == 0 || B == 0) return trc::usage("arguments faux");
    std::vector<uint64_t> dc(256, 0), cc(3 * 256, 0);
    Prepa p;
    for (uint32_t x = 0; x < n_experts; ++x) {
        preparer(blocs17[x], R, B, canon != 0, p);
        compter(p, dc.data(), cc.data());
    }
    normaliser(dc.data(), freqs4);
    for (int k = 0; k < 3; ++k) normaliser(cc.data() + 256 * k, freqs4 + 256 * (k + 1));
    return TRC_OK;
}

// One level-0 part of an expert (3 matrices). Returns the part length (multiple of 4096) and
// writes it to `out` when cap suffices; 0 on error.
namespace {
bool n_valides(const uint32_t* N_delta, const uint32_t* N_codes) {
    if (N_delta == nullptr || N_codes == nullptr) return false;
    for (int j = 0; j < 3; ++j)
        if (N_delta[j] == 0 || N_codes[j] == 0 || N_delta[j] > 65535 || N_codes[j] > 65535) return false;
    return true;
}
}  // namespace

uint64_t trc_codeur_partie(uint16_t couche, uint16_t expert, const trc_dims_expert* dims,
                           const uint8_t* const* blocs17, const float* const* biais, const uint16_t* const* freqs4,
                           int canon, uint32_t N_delta, uint32_t N_codes, uint8_t* out, uint64_t cap,
                           uint32_t* utiles) {
    const uint32_t nd[3] = {N_delta, N_delta, N_delta}, nc[3] = {N_codes, N_codes, N_codes};
    return trc_codeur_partie_n(couche, expert, dims, blocs17, biais, freqs4, canon, nd, nc, out, cap, utiles);
}

// The same with the tile lengths of each matrix j (N_delta[j], N_codes[j]): the format stores N per
// stream (decisions/ARCHITECTURE.md:581), so a part may mix them.
uint64_t trc_codeur_partie_n(uint16_t couche, uint16_t expert, const trc_dims_expert* dims,
                             const uint8_t* const* blocs17, const float* const* biais, const uint16_t* const* freqs4,
                             int canon, const uint32_t* N_delta, const uint32_t* N_codes, uint8_t* out, uint64_t cap,
                             uint32_t* utiles) {
    if (dims == nullptr || trc_dims_verifier(dims) != TRC_OK || !n_valides(N_delta, N_codes)) {
        trc::usage("dimensions ou N faux");
        return 0;
    }
    std::vector<FluxEcrit> flux;
    for (uint8_t j = 0; j < 3; ++j) {
        Prepa p;
        preparer(blocs17[j], dims->lignes[j], dims->colonnes[j] / 32, canon != 0, p);
        if (!coder_matrice(p, dims->lignes[j], biais[j], freqs4[j], j, N_delta[j], N_codes[j], flux)) {
            trc::usage("symbole absent de sa table (matrice %u)", j);
            return 0;
        }
    }
    uint32_t u;
    std::vector<uint8_t> b = assembler(couche, expert, 3, flux, u);
    if (utiles) *utiles = u;
    if (out && cap >= b.size()) std::memcpy(out, b.data(), b.size());
    return b.size();
}

// A whole synthetic layer: n experts generated from the seed, layer tables from counts over
// all of them (pass 1), parts coded with those tables (pass 2), n_fils threads.
trc_couche_synth* trc_synth_couche(uint64_t graine, uint32_t couche, uint32_t n_experts, const trc_dims_expert* dims,
                                   uint32_t N_delta, uint32_t N_codes, uint32_t n_fils) {
    const uint32_t nd[3] = {N_delta, N_delta, N_delta}, nc[3] = {N_codes, N_codes, N_codes};
    return trc_synth_couche_n(graine, couche, n_experts, dims, nd, nc, n_fils);
}

// The same with per-matrix tile lengths.
trc_couche_synth* trc_synth_couche_n(uint64_t graine, uint32_t couche, uint32_t n_experts,
                                     const trc_dims_expert* dims, const uint32_t* N_delta, const uint32_t* N_codes,
                                     uint32_t n_fils) {
    if (dims == nullptr || n_experts == 0 || trc_dims_verifier(dims) != TRC_OK || !n_valides(N_delta, N_codes)) {
        trc::usage("couche synthetique : arguments faux");
        return nullptr;
    }
    auto c = std::make_unique<trc_couche_synth>();
    const uint32_t B[3] = {dims->colonnes[0] / 32, dims->colonnes[1] / 32, dims->colonnes[2] / 32};
    auto tailles = [&](uint32_t j) { return size_t(dims->lignes[j]) * B[j] * 17; };
    // pass 1: counts per expert, then summed in expert order (integer sums: order-free)
    std::vector<std::vector<uint64_t>> comptes(n_experts, std::vector<uint64_t>(3 * 4 * 256, 0));
    en_parallele(n_experts, n_fils, [&](uint32_t e) {
        std::vector<uint8_t> bl[3];
        std::vector<float> bi[3];
        uint8_t* pb[3];
        float* pi[3];
        for (int j = 0; j < 3; ++j) {
            bl[j].resize(tailles(j));
            bi[j].resize(dims->lignes[j]);
            pb[j] = bl[j].data();
            pi[j] = bi[j].data();
        }
        trc_synth_expert(graine, couche, e, dims, pb, pi);
        Prepa p;
        for (int j = 0; j < 3; ++j) {
            preparer(pb[j], dims->lignes[j], B[j], true, p);
            compter(p, comptes[e].data() + 1024 * j, comptes[e].data() + 1024 * j + 256);
        }
    });
    for (int j = 0; j < 3; ++j) {
        std::vector<uint64_t> s(1024, 0);
        for (uint32_t e = 0; e < n_experts; ++e)
            for (int i = 0; i < 1024; ++i) s[i] += comptes[e][1024 * j + i];
        for (int t = 0; t < 4; ++t) normaliser(s.data() + 256 * t, c->freqs[j][t]);
    }
    // pass 2: regenerate and code
    c->parties.resize(n_experts);
    c->utiles.resize(n_experts);
    c->empreinte_origine.resize(n_experts);
    c->empreinte_canonique.resize(n_experts);
    std::atomic<bool> echec{false};
    en_parallele(n_experts, n_fils, [&](uint32_t e) {
        std::vector<uint8_t> bl[3];
        std::vector<float> bi[3];
        uint8_t* pb[3];
        float* pi[3];
        for (int j = 0; j < 3; ++j) {
            bl[j].resize(tailles(j));
            bi[j].resize(dims->lignes[j]);
            pb[j] = bl[j].data();
            pi[j] = bi[j].data();
        }
        trc_synth_expert(graine, couche, e, dims, pb, pi);
        c->empreinte_origine[e] = trc_empreinte_expert(pb, pi, dims);
        {
            std::vector<uint8_t> cb[3];
            const uint8_t* pc[3];
            for (int j = 0; j < 3; ++j) {
                cb[j] = bl[j];
                for (size_t q = 0; q < cb[j].size(); q += 17)
                    for (int t = 1; t < 17; ++t) cb[j][q + t] = canonique(cb[j][q + t]);
                pc[j] = cb[j].data();
            }
            c->empreinte_canonique[e] = trc_empreinte_expert(pc, pi, dims);
        }
        std::vector<FluxEcrit> flux;
        for (uint8_t j = 0; j < 3; ++j) {
            Prepa p;
            preparer(pb[j], dims->lignes[j], B[j], true, p);
            if (!coder_matrice(p, dims->lignes[j], pi[j], &c->freqs[j][0][0], j, N_delta[j], N_codes[j], flux))
                echec = true;
        }
        uint32_t u = 0;
        c->parties[e] = assembler(uint16_t(couche), uint16_t(e), 3, flux, u);
        c->utiles[e] = u;
    });
    if (echec) {
        trc::usage("couche synthetique : symbole absent de sa table");
        return nullptr;
    }
    return c.release();
}

uint64_t trc_synth_couche_empreinte(const trc_couche_synth* c, uint32_t e, int canon) {
    return canon ? c->empreinte_canonique[e] : c->empreinte_origine[e];
}
uint64_t trc_synth_couche_taille(const trc_couche_synth* c, uint32_t e) { return c->parties[e].size(); }
uint32_t trc_synth_couche_utiles(const trc_couche_synth* c, uint32_t e) { return c->utiles[e]; }
const uint8_t* trc_synth_couche_partie(const trc_couche_synth* c, uint32_t e) { return c->parties[e].data(); }
const uint16_t* trc_synth_couche_freqs(const trc_couche_synth* c) { return &c->freqs[0][0][0]; }
void trc_synth_couche_liberer(trc_couche_synth* c) { delete c; }

uint64_t trc_assembler_partie(uint16_t couche, uint16_t expert, uint8_t niveau, uint8_t n_matrices,
                              const trc_flux_a_ecrire* flux, uint32_t n, uint8_t* out, uint64_t cap,
                              uint32_t* utiles) {
    if (niveau > 1 || (n && flux == nullptr) || n > 65535) {
        trc::usage("assembler_partie : niveau %u, %u flux", niveau, n);
        return 0;
    }
    std::vector<FluxEcrit> v(n);
    for (uint32_t i = 0; i < n; ++i) {
        v[i].sorte = flux[i].sorte;
        v[i].matrice = flux[i].matrice;
        v[i].contexte = flux[i].contexte;
        v[i].produits = flux[i].produits;
        v[i].octets.assign(flux[i].octets, flux[i].octets + flux[i].longueur);
    }
    uint32_t u;
    const std::vector<uint8_t> b = assembler(couche, expert, n_matrices, v, u, niveau);
    if (utiles) *utiles = u;
    if (out && cap >= b.size()) std::memcpy(out, b.data(), b.size());
    return b.size();
}

int trc_synth_fichier(const char* chemin, uint64_t graine, uint16_t couches, uint16_t experts, uint16_t k,
                      const trc_dims_expert* dims, uint32_t N_delta, uint32_t N_codes, uint32_t n_fils,
                      uint64_t* taille) {
    if (chemin == nullptr || dims == nullptr || couches == 0 || experts == 0 || k == 0 || k > experts)
        return trc::usage("fichier synthetique : arguments faux");
    const int rd = trc_dims_verifier(dims);
    if (rd != TRC_OK) return rd;
    const uint32_t D = dims->colonnes[0];
    // MÉTA: gpt-oss-style hyper-parameters, then the encoder's additions (coder.rs:124-131)
    std::vector<uint8_t> meta;
    uint64_t n_paires = 0;
    auto cle = [&](const char* c, uint32_t type) {
        const uint64_t n = std::strlen(c);
        meta.insert(meta.end(), reinterpret_cast<const uint8_t*>(&n), reinterpret_cast<const uint8_t*>(&n) + 8);
        meta.insert(meta.end(), c, c + n);
        meta.insert(meta.end(), reinterpret_cast<const uint8_t*>(&type), reinterpret_cast<const uint8_t*>(&type) + 4);
        ++n_paires;
    };
    auto chaine = [&](const char* c, const char* v) {
        cle(c, 8);
        const uint64_t n = std::strlen(v);
        meta.insert(meta.end(), reinterpret_cast<const uint8_t*>(&n), reinterpret_cast<const uint8_t*>(&n) + 8);
        meta.insert(meta.end(), v, v + n);
    };
    auto u32 = [&](const char* c, uint32_t v) {
        cle(c, 4);
        meta.insert(meta.end(), reinterpret_cast<const uint8_t*>(&v), reinterpret_cast<const uint8_t*>(&v) + 4);
    };
    auto u64 = [&](const char* c, uint64_t v) {
        cle(c, 10);
        meta.insert(meta.end(), reinterpret_cast<const uint8_t*>(&v), reinterpret_cast<const uint8_t*>(&v) + 8);
    };
    chaine("general.architecture", "gpt-oss");
    chaine("general.name", "synthetique");
    u32("gpt-oss.block_count", couches);
    u32("gpt-oss.embedding_length", D);
    u32("gpt-oss.expert_feed_forward_length", dims->lignes[0]);
    u32("gpt-oss.expert_count", experts);
    u32("gpt-oss.expert_used_count", k);
    chaine("troncons.codeur.version", "troncons_amd codeur synthetique");
    chaine("troncons.source.nom", "synthetique");
    u64("troncons.synth.graine", graine);
    u32("troncons.synth.pas_delta", N_delta);
    u32("troncons.synth.pas_codes", N_codes);

    trc_ecrivain* w = trc_ecrivain_creer(chemin);
    if (w == nullptr) return TRC_FORMAT_ES;
    int r = trc_ecrivain_meta(w, meta.data(), meta.size(), n_paires);
    // RÉSIDENTS: the routers, bf16 rows of D values per expert
    std::vector<std::vector<uint8_t>> routeurs(couches);
    std::vector<trc_resident> res(couches);
    std::vector<const uint8_t*> donnees(couches);
    if (r == TRC_OK) {
        std::vector<float> ligne(D);
        for (uint32_t c = 0; c < couches; ++c) {
            routeurs[c].resize(size_t(experts) * D * 2);
            for (uint32_t e = 0; e < experts; ++e) {
                trc_synth_normale_bf16(graine + c, 3, e, D, 0.02f, ligne.data());
                for (uint32_t i = 0; i < D; ++i) {
                    uint32_t bits;
                    std::memcpy(&bits, &ligne[i], 4);
                    const uint16_t h = uint16_t(bits >> 16);  // the values are bf16-exact
                    std::memcpy(&routeurs[c][(size_t(e) * D + i) * 2], &h, 2);
                }
            }
            std::memset(&res[c], 0, sizeof(trc_resident));
            std::snprintf(res[c].nom, sizeof(res[c].nom), "blk.%u.ffn_gate_inp.weight", c);
            res[c].type_ggml = 30;  // GGML_TYPE_BF16
            res[c].n_dims = 2;
            res[c].ne[0] = D;
            res[c].ne[1] = experts;
            res[c].ne[2] = res[c].ne[3] = 1;
            res[c].octets = routeurs[c].size();
            donnees[c] = routeurs[c].data();
        }
        r = trc_ecrivain_residents(w, res.data(), donnees.data(), couches);
    }
    if (r == TRC_OK) r = trc_ecrivain_troncons(w, couches, experts);
    // TRONÇONS layer by layer; each layer's 12 tables are kept for the TABLES section
    std::vector<trc_table> tables;
    for (uint32_t c = 0; c < couches && r == TRC_OK; ++c) {
        trc_couche_synth* cs = trc_synth_couche(graine, c, experts, dims, N_delta, N_codes, n_fils);
        if (cs == nullptr) {
            r = TRC_ERREUR_USAGE;
            break;
        }
        for (uint32_t e = 0; e < experts && r == TRC_OK; ++e)
            r = trc_ecrivain_partie(w, uint16_t(c), uint16_t(e), cs->parties[e].data(), cs->parties[e].size(), nullptr,
                                    0, cs->empreinte_origine[e], cs->empreinte_canonique[e], nullptr);
        for (uint8_t j = 0; j < 3; ++j)
            for (int t = 0; t < 4; ++t) {
                trc_table tb;
                std::memset(&tb, 0, sizeof(tb));
                tb.couche = uint16_t(c);
                tb.matrice = j;
                tb.sorte = t == 0 ? trc::SORTE_DELTA : trc::SORTE_CODES_CTX;
                tb.contexte = uint8_t(t == 0 ? 0 : t - 1);
                tb.type_charge = 2;
                std::memcpy(tb.charge.frequences, cs->freqs[j][t], 512);
                tables.push_back(tb);
            }
        trc_synth_couche_liberer(cs);
    }
    if (r == TRC_OK) r = trc_ecrivain_tables(w, tables.data(), uint32_t(tables.size()));
    if (r != TRC_OK) {
        const std::string m = trc::derniere_erreur();
        trc_ecrivain_abandonner(w);
        trc::derniere_erreur() = m;
        return r;
    }
    trc_entete_fichier en;
    std::memset(&en, 0, sizeof(en));
    en.version_majeure = 1;
    en.version_mineure = 2;
    en.drapeaux = TRC_DRAPEAU_ALIGNE | TRC_DRAPEAU_CANONIQUE;
    trc_sha256(meta.data(), meta.size(), en.sha256_source);  // no source GGUF: the MÉTA pairs stand for it
    en.taille_source = 0;
    en.couches = couches;
    en.experts = experts;
    en.k = k;
    en.matrices = 3;
    for (int j = 0; j < 3; ++j) {
        en.lignes[j] = dims->lignes[j];
        en.colonnes[j] = dims->colonnes[j];
    }
    en.poids_par_bloc = 32;
    en.octets_par_bloc = 17;
    en.type_ggml = 39;
    en.niveaux = 1;
    en.classes_echelle = 3;
    return trc_ecrivain_terminer(w, &en, taille);
}

}  // extern "C"
