"""The expert slot cache and its simulator (csrc/cache.cpp through troncons_amd.cache).

Reference tests restated: moteur/crates/trc-cache/src/tests.rs (routage_fige_reponses_exactes
:63-79, epinglage_tient_les_k_experts_ensemble :90-125, en_vol_jamais_evince :128-135,
present_desepingle_est_evincable :138-150, deux_etages_egalent_deux_caches_a_pile :155-175,
belady_jamais_sous_lru :178-189, politique_faussee_donne_un_autre_compte :208-214,
lru_ordre_et_victime :216-229, trace_lue_comme_l_outil_python :231-240, trace_mal_formee_refusee
:242-249, octets_comptes_par_etage :252-273, belady_cas_calcule_a_la_main :279-286,
falaise_du_lru_global :294-306). Beyond them, the single-stage simulator is compared with a
pure-Python model written from the definitions (LRU and MIN that serve a whole group, then evict)
on random traces: hit counts and the final VRAM content must agree.
"""
from collections import OrderedDict

import numpy as np
import pytest

from troncons_amd import cache as K
from troncons_amd.cache import BELADY, DEFAUT_DISQUE, DEFAUT_RAM, FIFO, LRU, SUCCES, Cache, Trace, rejouer


class Alea:
    """splitmix64, for reproducible traces."""

    def __init__(self, g):
        self.e = g & 0xFFFFFFFFFFFFFFFF

    def suivant(self):
        self.e = (self.e + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = self.e
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        return z ^ (z >> 31)

    def sous(self, n):
        return self.suivant() % n

    def reel(self):
        return (self.suivant() >> 11) / float(1 << 53)


def trace_collante(t, l, e, k, rho, graine):
    """Sticky routing (tests.rs:24-53): each place keeps its expert with probability rho, else draws
    an expert absent from the current set."""
    a = Alea(graine)
    etat = []
    for _ in range(l):
        s = []
        while len(s) < k:
            x = a.sous(e)
            if x not in s:
                s.append(x)
        etat.append(s)
    choix = np.zeros((t, l, k), np.uint16)
    for j in range(t):
        for c, s in enumerate(etat):
            for i in range(k):
                if a.reel() >= rho:
                    while True:
                        x = a.sous(e)
                        if x not in s:
                            s[i] = x
                            break
            choix[j, c] = s
    return Trace.de(e, choix), choix


def trace_figee(t, l, k):
    choix = np.zeros((t, l, k), np.uint16)
    for c in range(l):
        choix[:, c] = np.arange(c, c + k)
    return Trace.de(32, choix)


def test_routage_fige_reponses_exactes():
    t, l, k = 4000, 4, 4
    tr = trace_figee(t, l, k)
    lk = l * k
    c0 = rejouer(tr, lk - k)
    assert c0.succes_vram == 0
    c1 = rejouer(tr, lk - 1)
    assert c1.succes_vram == (k - 1) * l * (t - 1)
    c2 = rejouer(tr, lk)
    assert c2.succes_vram == lk * (t - 1) and c2.evictions == 0
    for c in (c0, c1, c2):
        assert c.acces() == tr.acces()


def test_epinglage_tient_les_k_experts_ensemble():
    tr, choix = trace_collante(2000, 1, 12, 4, 0.5, 7)
    cache = Cache(4, 0)
    precedent = []
    for t in range(tr.jetons):
        g = list(choix[t, 0])
        d = cache.demander(0, g, 0)
        succes = sum(x.sorte == SUCCES for x in d)
        assert succes == sum(e in precedent for e in g), t
        precedent = g
        for i, e in enumerate(g):
            s = cache.emplacement_de(0, e)
            assert s is not None and s == d[i].emplacement and cache.occupant(s) == (0, e)
        for x in d:
            if x.sorte == DEFAUT_DISQUE:
                assert x.tiede is None
                cache.pret(x.emplacement)
        cache.liberer(0)


def test_en_vol_jamais_evince():
    cache = Cache(1, 0)
    cache.demander(0, [3], 0)
    cache.liberer(0)  # unpinned, but not `pret`
    with pytest.raises(K.ErreurUsage, match="aucun emplacement VRAM libre ni evincable"):
        cache.demander(1, [5], 1)


def test_present_desepingle_est_evincable():
    cache = Cache(1, 0)
    assert cache.demander(0, [3], 0) == [K.Decision(DEFAUT_DISQUE, 0, None)]
    assert cache.etat(0) == K.EN_VOL
    cache.pret(0)
    assert cache.etat(0) == K.PRESENT
    with pytest.raises(K.ErreurUsage):
        cache.pret(0)  # not in flight any more
    cache.liberer(0)
    assert cache.demander(1, [5], 1) == [K.Decision(DEFAUT_DISQUE, 0, None)]
    assert cache.compteurs().evictions == 1
    assert cache.etat(0) == K.EN_VOL and cache.occupant(0) == (1, 5) and cache.emplacement_de(0, 3) is None


def test_pinned_experts_are_never_victims():
    cache = Cache(4, 0)
    for x in cache.demander(0, [1, 2], 0):
        cache.pret(x.emplacement)
    assert sorted(cache.epingles()) == [(0, 1), (0, 2)]
    for x in cache.demander(1, [3, 4], 1):
        cache.pret(x.emplacement)
    with pytest.raises(K.ErreurUsage):  # 4 slots, 4 pinned (layers 0 and 1 still in progress)
        cache.demander(2, [5], 2)


@pytest.mark.parametrize("graine", range(4))
def test_deux_etages_egalent_deux_caches_a_pile(graine):
    tr, _ = trace_collante(800, 5, 32, 4, 0.55, 100 + graine)
    for v, r in [(8, 8), (8, 20), (16, 40), (30, 90), (12, 160)]:
        lru2 = rejouer(tr, v, r)
        assert lru2.succes_vram == rejouer(tr, v).succes_vram
        assert lru2.succes_vram + lru2.succes_ram == rejouer(tr, r).succes_vram
        assert lru2.acces() == tr.acces()
        b2 = rejouer(tr, v, r, BELADY, BELADY)
        assert b2.succes_vram == rejouer(tr, v, 0, BELADY, BELADY).succes_vram
        assert b2.succes_vram + b2.succes_ram == rejouer(tr, r, 0, BELADY, BELADY).succes_vram


def test_belady_jamais_sous_lru():
    for graine in range(6):
        tr, _ = trace_collante(600, 4, 64, 4, 0.3 + 0.1 * graine, graine)
        for n in (4, 8, 16, 33, 64, 128):
            assert rejouer(tr, n, 0, BELADY, BELADY).succes_vram >= rejouer(tr, n).succes_vram, (graine, n)


def test_politique_faussee_donne_un_autre_compte():
    tr, _ = trace_collante(1000, 4, 64, 4, 0.6, 3)
    assert rejouer(tr, 32).succes_vram != rejouer(tr, 32, 0, FIFO, FIFO).succes_vram


def test_lru_ordre_et_victime():
    cache = Cache(4, 0)
    for e in range(4):
        for x in cache.demander(0, [e], 0):
            cache.pret(x.emplacement)
        cache.liberer(0)
    cache.demander(0, [1], 1)
    cache.liberer(0)
    assert cache.ordre_vram() == [(0, 0), (0, 2), (0, 3), (0, 1)]
    # the victim is the oldest non-pinned: with (0, 0) pinned, (0, 2) goes
    d = cache.demander(0, [0, 9], 2)
    assert d[0].sorte == SUCCES and d[1].sorte == DEFAUT_DISQUE
    assert cache.emplacement_de(0, 2) is None and cache.ordre_vram() == [(0, 3), (0, 1), (0, 0), (0, 9)]


def test_trace_lue_comme_l_outil_python():
    tr = Trace.depuis_texte("# source\nE=32\n3 17 | 5 9\n\n3 31 | 5 2\n")
    assert (tr.experts, tr.couches, tr.k, tr.jetons) == (32, 2, 2, 2)
    assert tr.groupe(1, 0) == [3, 31] and tr.groupe(1, 1) == [5, 2]
    assert tr.commentaires == ["source"]
    assert Trace.depuis_texte("3 17 | 5 9").experts == 18


def test_trace_mal_formee_refusee():
    def err(texte):
        with pytest.raises(K.ErreurTrace) as e:
            Trace.depuis_texte(texte)
        return e.value
    e = err("1 2 | 3 4\n1 2\n")
    assert e.classe == "Ligne" and "ligne 2" in e.message
    e = err("1 2 | 3 4\n1 2 | 3\n")
    assert e.classe == "Ligne" and "ligne 2" in e.message
    e = err("E=4\n1 7\n")
    assert e.classe == "HorsBornes" and "7" in e.message and "4" in e.message
    assert err("# rien\n").classe == "Vide"
    e = err("1 x\n")
    assert e.classe == "Ligne" and "ligne 1" in e.message
    assert err("E=0\n1\n").classe == "Ligne"
    assert err("-1 2\n").classe == "Ligne"


def test_octets_comptes_par_etage():
    cache = Cache(1, 2)
    tailles = np.zeros((1, 4), np.uint64)
    tailles[0] = [1000, 1001, 1002, 1003]
    cache.fixer_tailles(tailles)
    for c, e in [(0, 1), (0, 2), (0, 1)]:
        for d in cache.demander(c, [e], 0):
            if d.sorte != SUCCES:
                cache.pret(d.emplacement)
        cache.liberer(c)
    k = cache.compteurs()
    assert (k.succes_vram, k.succes_ram, k.defauts_disque) == (0, 1, 2)
    assert k.octets_disque == 1001 + 1002
    assert k.octets_copies == 1001 + 1002 + 1001
    assert k.evictions == 2
    assert cache.tiede_de(0, 1) is not None and cache.tiede_de(0, 2) is not None


def test_ram_hit_decision_names_the_warm_entry():
    cache = Cache(1, 2)
    (d,) = cache.demander(0, [5], 0)
    assert d.sorte == DEFAUT_DISQUE and d.tiede == 0
    cache.pret(d.emplacement)
    cache.liberer(0)
    (d,) = cache.demander(0, [6], 1)
    assert d.sorte == DEFAUT_DISQUE and d.tiede == 1
    cache.pret(d.emplacement)
    cache.liberer(0)
    (d,) = cache.demander(0, [5], 2)
    assert d.sorte == DEFAUT_RAM and d.tiede == 0 and d.emplacement == 0


def test_belady_cas_calcule_a_la_main():
    tr = Trace.depuis_texte("E=3\n0\n1\n2\n0\n")
    assert rejouer(tr, 2, 0, BELADY, BELADY).succes_vram == 1
    assert rejouer(tr, 2).succes_vram == 0


@pytest.mark.parametrize("graine", range(4))
def test_falaise_du_lru_global(graine):
    l, k = 6, 4
    tr, _ = trace_collante(700, l, 16, k, 0.7, 40 + graine)
    seuil = (l - 1) * k
    for n in (k, 7, 13, seuil):
        assert rejouer(tr, n).succes_vram == 0, n
    assert rejouer(tr, seuil + 1).succes_vram > 0
    assert rejouer(tr, seuil, 0, BELADY, BELADY).succes_vram > 0


def test_belady_needs_the_trace():
    with pytest.raises(K.ErreurUsage):
        Cache(4, 0, BELADY, BELADY)


# ------------------------------------------------- an independent model from the definitions

def _lru_modele(choix, n):
    """LRU with an OrderedDict: serve the whole group (hits move to the newest end, misses enter),
    then evict the oldest until n remain."""
    od = OrderedDict()
    succes = 0
    t, l, k = choix.shape
    for j in range(t):
        for c in range(l):
            for e in choix[j, c]:
                cle = (c, int(e))
                if cle in od:
                    succes += 1
                    od.move_to_end(cle)
                else:
                    od[cle] = True
            while len(od) > n:
                od.popitem(last=False)
    return succes, list(od)


def _min_modele(choix, n):
    """MIN: serve the whole group, then evict, among the ids not in the current group, the one whose
    next use is farthest (never = infinity; ties: smallest (layer, expert))."""
    t, l, k = choix.shape
    usages = {}
    for j in range(t):
        for c in range(l):
            for e in choix[j, c]:
                v = usages.setdefault((c, int(e)), [])
                if not v or v[-1] != j * l + c:
                    v.append(j * l + c)
    present = set()
    succes = 0
    for j in range(t):
        for c in range(l):
            instant = j * l + c
            groupe = {(c, int(e)) for e in choix[j, c]}
            for e in choix[j, c]:
                if (c, int(e)) in present:
                    succes += 1
            present |= groupe
            while len(present) > n:
                def prochain(cle):
                    for u in usages[cle]:
                        if u > instant:
                            return u
                    return float("inf")
                cand = sorted(present - groupe, key=lambda x: (-prochain(x), x))
                present.remove(cand[0])
    return succes


@pytest.mark.parametrize("graine", range(5))
def test_simulator_equals_a_model_written_from_the_definitions(graine):
    rng = np.random.default_rng(graine)
    t, l, e, k = 300, 3, 10, 3
    choix = np.stack([np.stack([rng.choice(e, k, replace=False) for _ in range(l)]) for _ in range(t)])
    tr = Trace.de(e, choix)
    for n in (k, 5, 8, 12, 20):
        s, contenu = _lru_modele(choix, n)
        cache = Cache(n, 0)
        c = cache.rejouer_dans(tr)
        assert c.succes_vram == s, ("LRU", n)
        assert cache.ordre_vram() == contenu, ("LRU content", n)
        assert rejouer(tr, n, 0, BELADY, BELADY).succes_vram == _min_modele(choix, n), ("MIN", n)
