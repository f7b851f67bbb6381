"""CPU tests of the C-ABI library: it loads without a GPU, exports every declared symbol, its host
helpers give the reference's known answers (moteur/crates/trc-noyaux/src/abi.rs:303-407), its
encoder front-end writes exactly the oracle's bytes, and every launch wrapper refuses a contract
violation before touching the device (tests/carte.rs:468-479)."""
import ctypes as C
import pathlib
import re

import numpy as np
import pytest

import oracle_ffi as O
from troncons_amd import _lib, codeur
from troncons_amd import noyaux as K
from troncons_amd.noyaux import DimsExpert, VueCarte

RACINE = pathlib.Path(__file__).resolve().parents[1]


def _symboles_declares():
    noms = []
    for h in (RACINE / "include").glob("*.h"):
        texte = h.read_text()
        texte = re.sub(r"/\*.*?\*/", "", texte, flags=re.S)
        noms += re.findall(r"\b(trc_[a-z0-9_]+)\s*\(", texte)
    return sorted(set(noms))


def test_library_loads_and_exports_every_declared_symbol():
    l = _lib.charger()
    noms = _symboles_declares()
    assert len(noms) > 25
    manquants = [n for n in noms if not hasattr(l, n)]
    assert manquants == []


def test_struct_sizes_abi_rs_308():
    assert C.sizeof(DimsExpert) == 24 and C.alignment(DimsExpert) == 4
    assert C.sizeof(K.DescGemv) == 32
    assert C.sizeof(K.DescDecodage) == 32
    d = K.DescDecodage(1, 2 << 8, 3, 0xFFFFFFFFFFFFFFFF)
    o = d.octets()
    assert o[0] == 1 and o[9] == 2 and o[16] == 3 and o[24:32] == b"\xff" * 8


def test_slot_layout_and_grids_abi_rs_340():
    d = DimsExpert.gpt_oss()
    m = K.disposition_matrice(2880, 2880)
    assert (m.echelles, m.biais, m.pas) == (4_147_200, 4_406_528, 4_418_048)
    assert K.taille_emplacement(d) == 13_254_144
    assert K.disposition(d, 2).base == 2 * 4_418_048
    g1, g2 = K.grilles_decodeur(d)
    assert g1 == [2, 3, 1] and g2 == [16, 3, 1]
    assert K.grille_brut(d) == [96, 3, 1]
    with pytest.raises(K.ErreurUsage):
        K.verifier_dims(DimsExpert.de([2880] * 3, [2880, 2880, 100]))


def test_grids_read_from_part_abi_rs_362():
    p = bytearray(64 + 16 * 6 + 6 * 16)
    p[10] = 6
    for i, (sorte, j, t) in enumerate([(3, 0, 64), (4, 0, 127), (3, 1, 64), (4, 1, 127), (3, 2, 8), (4, 2, 127)]):
        e = 64 + 16 * i
        dec = 64 + 16 * 6 + 16 * i
        p[e] = sorte
        p[e + 1] = j
        p[e + 4:e + 8] = np.uint32(dec).tobytes()
        p[dec + 8:dec + 12] = np.uint32(t).tobytes()
    g1, g2 = K.grilles_depuis_partie(bytes(p))
    assert g1 == [16, 3, 1] and g2 == [16, 3, 1]
    p[64 + 16 * 5] = 0x01  # break: a missing stream is refused
    with pytest.raises(K.ErreurUsage):
        K.grilles_depuis_partie(bytes(p))


def test_lut_known_answers_abi_rs_385():
    f = np.zeros(256, np.uint16)
    f[3], f[200] = 4000, 96
    l = K.lut_geometrie1(f)
    assert l[0] == 3 | (3999 << 8) and l[3999] == 3 | (3999 << 8) | (3999 << 20)
    assert l[4000] == 200 | (95 << 8) and l[4095] == 200 | (95 << 8) | (95 << 20)
    f[3] = 3999
    with pytest.raises(K.ErreurUsage):
        K.lut_geometrie1(f)
    f = np.zeros(256, np.uint16)
    f[7] = 4096
    assert K.lut_geometrie1(f)[4095] == 7 | (4095 << 8) | (4095 << 20)


def test_luts_couche_equals_oracle():
    rng = np.random.default_rng(1)
    tables = [[None] * 4 for _ in range(3)]
    for j in range(3):
        for t in range(4):
            if (j, t) != (1, 2):
                c = rng.integers(0, 1000, 256).astype(np.uint64)
                tables[j][t] = O.table_depuis_comptes(c)
    assert (K.luts_couche(tables) == O.luts_couche(tables)).all()


# ------------------------------------------------------------------------ encoder front-end

def test_generators_equal_the_oracle():
    bl, bi = codeur.synth_matrice(77, 3, 5, 2, 64, 320)
    ob, oi = O.synth_matrice(77, 3, 5, 2, 64, 320)
    assert (bl == ob).all() and (bi.view(np.uint32) == oi.view(np.uint32)).all()
    assert (codeur.synth_normale_bf16(9, 1, 2, 1001, 1.0).view(np.uint32) ==
            O.synth_normale_bf16(9, 1, 2, 1001, 1.0).view(np.uint32)).all()


def _experts(dims, n, graine=5):
    return [codeur.synth_expert(graine, 0, e, dims) for e in range(n)]


@pytest.mark.parametrize("N", [(256, 256), (16, 32), (3, 5)])
def test_encoder_writes_the_oracle_bytes(N):
    dims = DimsExpert.de([96, 96, 64], [320, 320, 96])
    ex = _experts(dims, 3)
    for j in range(3):
        R, B = dims.lignes[j], dims.colonnes[j] // 32
        t = codeur.tables([e[0][j] for e in ex], R, B)
        assert (t == O.tables_matrice([e[0][j] for e in ex], R, B, canonique=True)).all()
    freqs = [codeur.tables([e[0][j] for e in ex], dims.lignes[j], dims.colonnes[j] // 32) for j in range(3)]
    for x, (bl, bi) in enumerate(ex):
        p, u = codeur.partie(bl, bi, freqs, dims, expert=x, N_delta=N[0], N_codes=N[1])
        po, uo = O.coder_expert(bl, bi, list(dims.lignes), list(dims.colonnes), freqs, expert=x, canonique=True,
                                N_delta=N[0], N_codes=N[1])
        assert u == uo and p == po


def test_synthetic_layer_equals_per_expert_encoding():
    dims = DimsExpert.de([64] * 3, [256] * 3)
    couche = codeur.CoucheSynthetique(11, 2, 4, dims, N_delta=8, N_codes=16, n_fils=3)
    ex = [codeur.synth_expert(11, 2, e, dims) for e in range(4)]
    freqs = [codeur.tables([e[0][j] for e in ex], 64, 8) for j in range(3)]
    assert (couche.freqs() == np.stack(freqs)).all()
    for e in range(4):
        p, u = codeur.partie(ex[e][0], ex[e][1], freqs, dims, couche=2, expert=e, N_delta=8, N_codes=16)
        assert couche.utiles(e) == u and bytes(couche.partie(e)) == p
    couche.liberer()


def test_synthetic_expert_deinterleaves_gate_up():
    dims = DimsExpert.de([32] * 3, [64] * 3)
    bl, bi = codeur.synth_expert(3, 1, 7, dims)
    gu, bgu = O.synth_matrice(3, 1, 7, 1, 64, 64)
    gu = gu.reshape(64, 2 * 17)
    assert (bl[0].reshape(32, -1) == gu[0::2]).all() and (bl[1].reshape(32, -1) == gu[1::2]).all()
    assert (bi[0] == bgu[0::2]).all() and (bi[1] == bgu[1::2]).all()
    dn, bdn = O.synth_matrice(3, 1, 7, 2, 32, 64)
    assert (bl[2] == dn).all() and (bi[2] == bdn).all()


# ------------------------------------------------------------- wrappers refuse before launching

def test_wrappers_refuse_wrong_sizes_carte_rs_468():
    k = K.Noyaux()
    dims = DimsExpert.gpt_oss()
    petit = VueCarte(1 << 20, 4096)
    with pytest.raises(K.ErreurUsage):
        k.decoder_expert(petit, petit, petit, dims, petit, f=0)
    with pytest.raises(K.ErreurUsage):
        k.gemv(petit, petit, petit, 2880, 2880, f=0)
    with pytest.raises(K.ErreurUsage):
        k.gemv(VueCarte(1 << 20, 10 ** 8), VueCarte(16, 4 * 2880), VueCarte(32, 4 * 2880), 2880, 2880 + 1, f=0)
    with pytest.raises(K.ErreurUsage):  # x not 16-aligned
        k.gemv(VueCarte(1 << 20, 10 ** 8), VueCarte(8, 4 * 2880), VueCarte(32, 4 * 2880), 2880, 2880, f=0)
    with pytest.raises(K.ErreurUsage):  # slot not 256-aligned
        k.decoder_expert(VueCarte(64, 4096), VueCarte(128, 13_254_144), VueCarte(1 << 20, 3 * 4 * 4096 * 4), dims,
                         VueCarte(1 << 12, 16), f=0)
    with pytest.raises(K.ErreurUsage):
        k.routeur_topk(petit, 300, 4, petit, petit, f=0)
    with pytest.raises(K.ErreurUsage):
        k.combiner(petit, petit, 10, None, 4, 2880, f=0)
    with pytest.raises(K.ErreurUsage):
        k.decoder_lot(petit, 0, dims, f=0)
    assert "usage" in K.bibliotheque().trc_derniere_erreur().decode()


def test_prefill_refuses_unsupported_shapes_before_launching():
    """The batched prefill keeps a row's blocks in LDS (at most 4096 columns) and at most 16384
    (position, slot) pairs a call: other shapes are usage errors, returned before any HIP call. Any
    CODES_CTX tile length is taken: below 16 macro-steps the band kernels decode their tiles, tiles
    of 16 or more (the bench's 16 and 32, the reference encoder's 256, rans.rs:32) are decoded once
    per chosen expert into a slot of the reference layout, which the workspace then holds for every
    expert of the layer."""
    from troncons_amd import fusion

    fz = fusion.Fusion()
    dims = DimsExpert.gpt_oss()
    v = VueCarte(1 << 20, 1 << 40)
    court = fusion.taille_travail_prefill(dims, 128, 512, 4, 8)
    assert court > 0
    for n in (16, 17, 32, 256):
        long_ = fusion.taille_travail_prefill(dims, 128, 512, 4, n)
        assert long_ > court and long_ >= 128 * K.taille_emplacement(dims)
    assert fusion.taille_travail_prefill(dims, 128, 512, 4, 0) == 0
    assert fusion.taille_travail_prefill(DimsExpert.de([256, 256, 256], [8192, 8192, 256]), 8, 4, 4, 8) == 0
    assert fusion.taille_travail_prefill(dims, 128, 8192, 4, 16) == 0  # more than 16384 pairs
    with pytest.raises(K.ErreurUsage):
        fz.prefill_moe(v, 128, v, dims, v, 512, v, v, 4, v, v, v, 4, 0, f=0)
    with pytest.raises(K.ErreurUsage):  # workspace too small
        fz.prefill_moe(v, 128, v, dims, v, 512, v, v, 4, v, v, VueCarte(1 << 20, 4096), 4, 16, f=0)
    with pytest.raises(K.ErreurUsage):  # long tiles: the slots do not fit a short-tile workspace
        fz.prefill_moe(v, 128, v, dims, v, 512, v, v, 4, v, v, VueCarte(1 << 20, court), 256, 256, f=0)


def test_driver_half_refuses_bad_arguments_before_any_hip_call():
    """The driver half's contract checks (trc-cuda/src/lib.rs:448-451, 521-524, 591-623) run before
    the runtime is touched, so they answer without a device."""
    l = K.bibliotheque()  # declared return types: the error text is a char pointer
    from troncons_amd import pilote  # noqa: F401  (declares the argument types)
    V = K._Vue
    h = C.c_void_p()
    assert l.trc_contexte_creer(0, 9, C.byref(h)) == 1 and b"attente" in l.trc_derniere_erreur()
    assert l.trc_dernier_code_hip() == 0
    assert l.trc_carte_remplir(V(0, 16), 0, None) == 1
    assert l.trc_carte_remplir(V(0, 0), 0, None) == 0  # an empty view is nothing to do
    assert l.trc_copier_carte_carte(V(4096, 4), V(8192, 8), None) == 1
    assert l.trc_copier_vers_carte(V(4096, 4), None, 4, None) == 1
    assert l.trc_copier_vers_carte(V(4096, 4), C.c_void_p(8192), 8, None) == 1
    assert l.trc_copier_vers_hote(None, V(4096, 4), None) == 1
    assert l.trc_flux_attendre(None, None) == 1
    assert l.trc_evenement_ms_depuis(None, None, None) == 1
    assert l.trc_hote_allouer(None, 0, 0, C.byref(h), None, None) == 1
    assert l.trc_carte_allouer(None, 0, C.byref(V())) == 1


def test_streamed_layer_engine_refuses_bad_arguments_before_any_hip_call():
    """trc_diffusion_creer and trc_diffusion_couche check their arguments before the runtime is
    touched: no layers, a top-k above the experts or above 8, shapes the fused path refuses, parts
    not 16-byte aligned, a router too short, a null engine."""
    from troncons_amd import diffusion as Df
    l = Df._l()
    dims = DimsExpert.gpt_oss()
    E, k = 8, 4
    dec = (C.c_uint64 * E)(*[4096 * e for e in range(E)])
    tai = (C.c_uint64 * E)(*([4096] * E))
    V = K._Vue
    luts, routeur = V(1 << 20, 4 * 3 * 4 * 4096), V(1 << 24, 4 * E * 2880)
    bonne = Df.CoucheHote(1 << 30, dec, tai, luts, routeur)
    h = C.c_void_p()

    def creer(couches, n, experts=E, kk=k, d=dims, nd=1, nc=16):
        return l.trc_diffusion_creer(couches, n, experts, kk, C.byref(d), nd, nc, C.byref(h))

    tab = (Df.CoucheHote * 1)(bonne)
    assert creer(None, 0) == 1
    assert creer(tab, 1, kk=0) == 1
    assert creer(tab, 1, kk=9, experts=16) == 1
    assert creer(tab, 1, experts=3, kk=4) == 1
    assert creer(tab, 1, d=DimsExpert.de([2880, 2880, 2880], [2880, 2880, 2048])) == 1
    assert creer(tab, 1, nc=0) == 1
    mal = (Df.CoucheHote * 1)(Df.CoucheHote((1 << 30) + 8, dec, tai, luts, routeur))
    assert creer(mal, 1) == 1 and b"align" in l.trc_derniere_erreur()
    court = (Df.CoucheHote * 1)(Df.CoucheHote(1 << 30, dec, tai, luts, V(1 << 24, 16)))
    assert creer(court, 1) == 1 and b"routeur" in l.trc_derniere_erreur()
    assert h.value is None
    assert l.trc_diffusion_couche(None, 0, V(1 << 20, 4 * 2880), V(1 << 21, 4 * 2880), None, None) == 1
    assert l.trc_diffusion_jeton(None, V(1 << 20, 4 * 2880), V(1 << 21, 4 * 2880), None) == 1
