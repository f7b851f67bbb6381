"""The native streaming scheduler (csrc/ordo.cpp) on the GPU: tokens through every layer of a .trc
file with the experts streamed from disk and kept decoded in a slot cache in HBM.

Checked, as the reference checks its engine (trc-ordo, trc-cache witness O3):
- per token, the residual equals the oracle's chain — router and top-k on x, each chosen expert's
  part decoded by the oracle, the reference GEMV order, swiglu_oai, the ordered combine — within
  1e-5 * max|r| (the reference's GEMV threshold), and the routing the engine saw equals the oracle's
  top-k exactly;
- the engine's cache counters (hits per stage, misses, evictions, bytes) equal the simulator's
  replay of the engine's own routing trace, to the unit, and its read and copy byte counts equal
  the counters' bytes;
- every expert still decoded in a VRAM slot hashes to the directory's canonical fingerprint;
- a part damaged on disk is refused by the fingerprint check when reads are checked, and counted
  in the control words by the decoder when they are not.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle_ffi as O  # noqa: E402
from gpu_outils import dev, hote, zeros  # noqa: E402
from troncons_amd import cache as K  # noqa: E402
from troncons_amd import conteneur as T  # noqa: E402
from troncons_amd.noyaux import DimsExpert, ErreurUsage  # noqa: E402
from troncons_amd.ordo import Ordonnanceur  # noqa: E402

TOL = 1e-5


class Modele:
    """A small synthetic model file and the oracle's view of it."""

    def __init__(self, chemin, graine, L, E, k, dims, N=(4, 16)):
        T.synth_fichier(chemin, graine, L, E, k, dims, N_delta=N[0], N_codes=N[1], n_fils=16)
        self.f = T.Fichier.ouvrir(chemin)
        self.chemin, self.graine, self.L, self.E, self.k, self.dims = chemin, graine, L, E, k, dims
        self.luts = [O.luts_couche(self.f.freqs_couche(l)) for l in range(L)]
        self.routeurs = []
        for l in range(L):
            (r,) = [r for r in self.f.residents() if r.nom == f"blk.{l}.ffn_gate_inp.weight"]
            r16 = self.f.donnees_resident(r).view(np.uint16).reshape(E, -1)
            self.routeurs.append((r16.astype(np.uint32) << 16).view(np.float32))
        self._slots = {}

    def slot(self, l, e):
        if (l, e) not in self._slots:
            p = self.f.lire_partie(l, e).tobytes()
            s, ctl = O.decoder_expert(p, self.luts[l], list(self.dims.lignes), list(self.dims.colonnes))
            assert (ctl == 0).all()
            self._slots[(l, e)] = s
        return self._slots[(l, e)]

    def jeton(self, x, choisir=None):
        """The oracle chain of one token; `choisir(l, logits)` -> (indices, weights) replaces the
        plain top-k (the biased router's replay)."""
        lg, cl = list(self.dims.lignes), list(self.dims.colonnes)
        R, C, D = lg[0], cl[0], lg[2]
        d = [O.disposition_j(lg, cl, j) for j in range(3)]
        residu = np.zeros(D, np.float32)
        choix = []
        for l in range(self.L):
            logits = O.gemv_f32(self.routeurs[l], x)
            oi, ow = choisir(l, logits) if choisir else O.routeur_topk(logits, self.k)
            choix.append(oi)
            sorties = []
            for e in oi:
                s = self.slot(l, int(e))
                g = O.gemv_mxfp4(s[d[0].base:d[0].base + d[0].pas], x, R, C)
                u = O.gemv_mxfp4(s[d[1].base:d[1].base + d[1].pas], x, R, C)
                a = O.swiglu_oai(g, u)
                sorties.append(O.gemv_mxfp4(s[d[2].base:d[2].base + d[2].pas], a, D, R))
            residu = O.combiner(residu, np.concatenate(sorties), D, ow, self.k, D)
        return residu, np.array(choix)


def _tokens(graine, n, C):
    return [O.synth_normale_bf16(graine, 4, t, C, 1.0) for t in range(n)]


def _run(m, o, xs, verifier_residus=True):
    D = m.dims.lignes[2]
    for t, x in enumerate(xs):
        print(f"token {t}", flush=True)
        xd, res = dev(x), zeros(4 * D)
        o.jeton(xd, res)
        got = hote(res, np.float32)
        if verifier_residus:
            ref, choix = m.jeton(x)
            assert (o.trace()[t] == choix).all(), t
            assert np.abs(got - ref).max() <= TOL * np.abs(ref).max(), t
    assert list(o.controle()) == [0, 0, 0, 0]


def _temoins(m, o, emplacements, tiedes):
    c = o.compteurs()
    tr = o.trace()
    sim = K.Cache(emplacements, tiedes)
    sim.fixer_tailles(np.array([[m.f.entree(l, e).longueur[0] for e in range(m.E)] for l in range(m.L)], np.uint64))
    s = sim.rejouer_dans(K.Trace.de(m.E, tr))
    assert c.tuple() == s.tuple()
    assert c.acces() == tr.size
    st = o.stats()
    assert st.octets_lus == c.octets_disque and st.octets_copies == c.octets_copies
    assert st.decodages == c.defauts_disque + c.succes_ram and st.lectures == c.defauts_disque
    vus = 0
    for l in range(m.L):
        for e in range(m.E):
            h = o.temoin(l, e)
            if h is not None:
                assert h == m.f.entree(l, e).empreinte_canonique, (l, e)
                vus += 1
    assert vus == min(emplacements, len({(l, int(e)) for l in range(m.L) for e in np.unique(tr[:, l])}))
    return c


@pytest.fixture(scope="module")
def petit(tmp_path_factory):
    assert torch.cuda.is_available()
    d = DimsExpert.de([256, 256, 256], [256, 256, 256])
    return Modele(tmp_path_factory.mktemp("ordo") / "petit.trc", 2030, 4, 16, 4, d)


def test_engine_with_both_stages_equals_oracle_and_simulator(petit):
    # the RAM stage is inclusive: it only serves hits when it is larger than the VRAM stage
    o = Ordonnanceur(petit.f, emplacements=24, tiedes=40, verifier=True)
    _run(petit, o, _tokens(2030, 30, 256))
    c = _temoins(petit, o, 24, 40)
    assert c.succes_vram > 0 and c.succes_ram > 0 and c.defauts_disque > 0 and c.evictions > 0 and c.evictions_ram > 0
    o.detruire()


def test_engine_without_ram_stage_minimum_slots(petit):
    o = Ordonnanceur(petit.f, emplacements=4, tiedes=0, verifier=False, lecteurs=2)
    _run(petit, o, _tokens(2031, 12, 256))
    c = _temoins(petit, o, 4, 0)
    assert c.succes_ram == 0 and c.evictions > 0
    o.detruire()


def test_engine_all_experts_resident_after_warmup(petit):
    o = Ordonnanceur(petit.f, emplacements=64, tiedes=0)
    xs = _tokens(2032, 40, 256)
    _run(petit, o, xs, verifier_residus=False)
    c = _temoins(petit, o, 64, 0)
    assert c.evictions == 0 and c.defauts_disque == len({(l, int(e)) for l in range(4) for e in np.unique(o.trace()[:, l])})
    # a second pass over the same tokens is all VRAM hits and still equals the oracle
    avant = o.compteurs().succes_vram
    _run(petit, o, xs[:5])
    assert o.compteurs().succes_vram == avant + 5 * 4 * 4
    o.detruire()


def test_damaged_part_refused_or_counted(petit, tmp_path):
    b = bytearray(petit.chemin.read_bytes())
    en = petit.f.entree(0, 3)
    p = T.lire_partie(np.frombuffer(bytes(b[en.decalage:en.decalage + en.longueur[0]]), np.uint8))
    codes = p.trouver(T.SORTE_CODES_CTX, 0)
    b[en.decalage + codes.decalage + codes.longueur // 2] ^= 0x5A
    chemin = tmp_path / "abime.trc"
    chemin.write_bytes(bytes(b))
    f = T.Fichier.ouvrir(chemin)  # parts are not read at opening
    # every expert of layer 0 is asked for over a few tokens with 16 slots: expert 3 is read
    xs = _tokens(2033, 24, 256)
    vus = set()
    for t, x in enumerate(xs):
        oi, _ = O.routeur_topk(O.gemv_f32(petit.routeurs[0], x), 4)
        vus |= set(int(e) for e in oi)
        if 3 in vus:
            n = t + 1
            break
    else:
        pytest.skip("expert (0, 3) never routed on these tokens")
    o = Ordonnanceur(f, emplacements=64, tiedes=0, verifier=True)
    with pytest.raises(T.ErreurFormat) as e:
        for x in xs[:n]:
            o.jeton(dev(x), zeros(4 * 256))
    assert e.value.classe == "Empreinte"
    # fail-stop: the failed token's reads were drained and every later token is refused
    with pytest.raises(ErreurUsage, match="erreur precedente"):
        o.jeton(dev(xs[0]), zeros(4 * 256))
    o.detruire()
    o = Ordonnanceur(f, emplacements=64, tiedes=0, verifier=False)
    for x in xs[:n]:
        o.jeton(dev(x), zeros(4 * 256))
    assert o.controle().sum() > 0
    o.detruire()


def test_engine_gpt_oss_shape(tmp_path_factory):
    m = Modele(tmp_path_factory.mktemp("ordo") / "gpt.trc", 2034, 2, 8, 4, DimsExpert.gpt_oss())
    o = Ordonnanceur(m.f, emplacements=10, tiedes=4, verifier=True)
    xs = _tokens(2034, 3, 2880)
    _run(m, o, xs[:1])
    _run(m, o, xs[1:], verifier_residus=False)
    _temoins(m, o, 10, 4)
    o.detruire()


@pytest.fixture(scope="module")
def deux(tmp_path_factory):
    d = DimsExpert.de([256, 256, 256], [256, 256, 256])
    return Modele(tmp_path_factory.mktemp("ordo2") / "deux.trc", 2032, 2, 16, 4, d)


def test_prefetch_reads_ahead_and_changes_no_result(deux):
    """Config::prechargement (trc-ordo/src/lib.rs:1104-1215, trc-modele/src/lib.rs:570-579): layer 0
    predicts layer 1's experts with layer 1's router over the residual normed with layer 1's
    post-attention norm (unit weights: the file holds none), and the predicted parts are read ahead.
    The router input x is taken as that same norm of the incoming residual, so the prediction is
    layer 1's routing: every part read ahead serves a disk miss of layer 1 (on the first token, with
    an empty cache, all k of them). Residuals are bit-identical with and without prefetch, the
    cache counters equal each other and the simulator's replay, and every read is accounted for."""
    from troncons_amd.noyaux import Noyaux
    m = deux
    D, C = m.dims.lignes[2], m.dims.colonnes[0]
    n = Noyaux()
    un = dev(np.ones(D, np.float32))
    a = Ordonnanceur(m.f, emplacements=8, tiedes=0, verifier=True)
    b = Ordonnanceur(m.f, emplacements=8, tiedes=0, verifier=True, prechargement=True)
    for t in range(8):
        print(f"token {t}", flush=True)
        r0 = O.synth_normale_bf16(2033, 5, t, D, 3.0)
        x = zeros(4 * C)
        n.rmsnorm(dev(r0), un, x, D, 1, 1e-5)
        ra, rb = dev(r0), dev(r0)
        a.jeton(x, ra)
        b.jeton(x, rb)
        assert (hote(ra, np.uint32) == hote(rb, np.uint32)).all(), t
        if t == 0:
            assert b.stats().pf_utiles == b.stats().pf_emis == m.k
    assert (a.trace() == b.trace()).all()
    assert list(b.controle()) == [0, 0, 0, 0]
    sa, sb = a.stats(), b.stats()
    assert sa.pf_emis == sa.pf_utiles == sa.pf_octets == 0
    ca, cb = a.compteurs(), b.compteurs()
    assert ca.tuple() == cb.tuple()
    # every read ahead was used: the same parts and bytes are read, layer 1's a layer earlier
    assert sb.pf_utiles == sb.pf_emis > m.k
    assert sb.lectures == cb.defauts_disque - sb.pf_utiles + sb.pf_emis == sa.lectures
    assert sb.octets_lus == sa.octets_lus == ca.octets_disque and 0 < sb.pf_octets < sb.octets_lus
    assert sb.octets_copies == sa.octets_copies and sb.decodages == sa.decodages
    _temoins_cache(m, b, 8, 0)


def _temoins_cache(m, o, emplacements, tiedes):
    """The cache counters against the simulator's replay of the engine's trace, and the decoded
    slots against the canonical fingerprints (reads are not compared: prefetch adds its own)."""
    c = o.compteurs()
    tr = o.trace()
    sim = K.Cache(emplacements, tiedes)
    sim.fixer_tailles(np.array([[m.f.entree(l, e).longueur[0] for e in range(m.E)] for l in range(m.L)], np.uint64))
    assert c.tuple() == sim.rejouer_dans(K.Trace.de(m.E, tr)).tuple()
    for l in range(m.L):
        for e in range(m.E):
            h = o.temoin(l, e)
            if h is not None:
                assert h == m.f.entree(l, e).empreinte_canonique, (l, e)


def test_cache_biased_router_replays_exactly(petit):
    """Config::biais_cache (trc-ordo/src/lib.rs:1089-1100): before layer l's request the engine adds
    beta to the router score of each of l's experts in a VRAM slot. Replayed in lockstep with the
    cache mirror (the same decisions, pret, liberer) and the oracle's biased top-k, the engine's
    routing is the replay's, exactly, and its residual is the oracle chain's over those choices
    within 1e-5 * max|r|; beta = 0 gives the plain engine's bits; a positive beta raises the VRAM
    hit rate on the same tokens (24 slots: a token's experts are still resident at the next token, so
    there is something for the bias to prefer)."""
    m = petit
    D = m.dims.lignes[2]
    xs = _tokens(2034, 8, m.dims.colonnes[0])
    plain = Ordonnanceur(m.f, emplacements=24, tiedes=0)
    zero = Ordonnanceur(m.f, emplacements=24, tiedes=0, biais_cache=0.0)
    biased = Ordonnanceur(m.f, emplacements=24, tiedes=0, biais_cache=1.0)
    sim = K.Cache(24, 0)
    sim.fixer_tailles(np.array([[m.f.entree(l, e).longueur[0] for e in range(m.E)] for l in range(m.L)], np.uint64))
    for t, x in enumerate(xs):
        print(f"token {t}", flush=True)
        rp, rz, rb = zeros(4 * D), zeros(4 * D), zeros(4 * D)
        xd = dev(x)
        plain.jeton(xd, rp)
        zero.jeton(xd, rz)
        biased.jeton(xd, rb)
        assert (hote(rp, np.uint32) == hote(rz, np.uint32)).all(), t

        def choisir(l, logits, t=t):
            b = np.array([1.0 if sim.emplacement_de(l, e) is not None else 0.0 for e in range(m.E)], np.float32)
            oi, ow = O.routeur_topk_biais(logits, b, m.k)
            for dcs in sim.demander(l, oi, t * m.L + l):
                if dcs.sorte != K.SUCCES:
                    sim.pret(dcs.emplacement)
            sim.liberer(l)
            return oi, ow

        ref, choix = m.jeton(x, choisir)
        assert (biased.trace()[t] == choix).all(), t
        got = hote(rb, np.float32)
        assert np.abs(got - ref).max() <= TOL * np.abs(ref).max(), t
    assert (plain.trace() == zero.trace()).all()
    assert biased.compteurs().tuple() == sim.compteurs().tuple()
    assert biased.compteurs().succes_vram > plain.compteurs().succes_vram
    assert list(biased.controle()) == [0, 0, 0, 0]
    for cfg in ({"biais_cache": float("inf")}, {"biais_cache": 1.0, "prechargement": True}):
        with pytest.raises(Exception):
            Ordonnanceur(m.f, emplacements=24, tiedes=0, **cfg)
