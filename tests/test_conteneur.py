"""The .trc v1.2 container (csrc/conteneur.cpp through troncons_amd.conteneur) against the
reference's own container tests and what the format fixes.

Reference tests followed: moteur/crates/trc-format/tests/aller_retour.rs (aller_retour_identique
:181-226, cassures_refusees :238-289, aller_retour_v12_canonique :303-327, cassures_v12_refusees
:329-372, drapeau_rapide_v12 :376-401, temoin_du_temoin :403-413, empreinte64_connue :411-416).
SHA-256 is pinned against Python's hashlib (an independent implementation) over lengths that cross
every padding boundary. Beyond the reference: each refusal class is reached by a targeted, re-hashed
change, so a check that is dropped or misclassified fails; and a synthetic model file is checked
against the encoder's parts and tables, hashlib fingerprints of the generated experts, and the CPU
oracle's decode of the parts read back from disk.
"""
import hashlib
import struct

import numpy as np
import pytest

import oracle_ffi as O
from troncons_amd import DimsExpert
from troncons_amd import codeur
from troncons_amd import conteneur as T
from troncons_amd.conteneur import ErreurFormat


def _classe(fn):
    with pytest.raises(ErreurFormat) as e:
        fn()
    return e.value.classe


# ------------------------------------------------------------------------------ fingerprints

def test_empreinte64_known_answer_aller_retour_411():
    assert T.empreinte64(b"abc") == int.from_bytes(bytes([0xBA, 0x78, 0x16, 0xBF, 0x8F, 0x01, 0xCF, 0xEA]), "little")
    assert T.empreinte64_morceaux([b"a", b"bc"]) == T.empreinte64(b"abc")


def test_sha256_equals_hashlib_across_padding_boundaries():
    rng = np.random.default_rng(1)
    longueurs = list(range(0, 200)) + [447, 448, 449, 511, 512, 513, 4095, 4096, 4097, 1 << 20]
    for n in longueurs:
        b = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        h = hashlib.sha256(b).digest()
        assert T.sha256(b) == h, n
        assert T.empreinte64(b) == int.from_bytes(h[:8], "little"), n
    # the oracle's restatement agrees too
    b = rng.integers(0, 256, 100_003, dtype=np.uint8).tobytes()
    assert O.empreinte64(b) == T.empreinte64(b)


def test_canonisation_aller_retour_366():
    assert sum(T.porte_un_8(o) for o in range(256)) == 31
    assert T.canoniser_octet(0x88) == 0x00
    assert T.canoniser_octet(0x8F) == 0x0F
    assert T.canoniser_octet(0x78) == 0x70
    assert all(not T.porte_un_8(T.canoniser_octet(o)) and (T.porte_un_8(o) or T.canoniser_octet(o) == o)
               for o in range(256))


# --------------------------------------------------------------------- the reference's file

def _paire_u32(cle, v):
    c = cle.encode()
    return len(c).to_bytes(8, "little") + c + (4).to_bytes(4, "little") + v.to_bytes(4, "little")


def _paire_tableau_chaines(cle, elems):
    c = cle.encode()
    b = len(c).to_bytes(8, "little") + c + (9).to_bytes(4, "little") + (8).to_bytes(4, "little")
    b += len(elems).to_bytes(8, "little")
    for s in elems:
        e = s.encode()
        b += len(e).to_bytes(8, "little") + e
    return b


class Construit:
    pass


def _ecrire(chemin, canonique=False, table_8=False, tables_apres=False):
    """The small complete file of aller_retour.rs:80-178: MÉTA with a string, a u32, an array of
    strings and one added pair; three residents of unaligned sizes; DELTA and CODES_CTX tables per
    (layer, matrix) written out of order, plus a COMPL_CTX and a CENTRES table; 2 x 3 parts of 12
    random streams. ``tables_apres`` writes TABLES after the parts instead."""
    rng = np.random.default_rng(0x9E3779B97F4A7C15 & 0xFFFFFFFF)
    c = Construit()
    w = T.Ecrivain(chemin)
    brute = T.paire_chaine("general.architecture", "essai") + _paire_u32("essai.couches_x", 2) + \
        _paire_tableau_chaines("jetons", ["a", "été"])
    ajout = T.paire_chaine("troncons.codeur.version", "essai")
    w.meta(brute + ajout, 4)
    c.meta_brute = (4).to_bytes(8, "little") + brute + ajout

    tailles = [1000, 34 * 5, 4 * 3]
    c.donnees = [rng.integers(0, 256, t, dtype=np.uint8).tobytes() for t in tailles]
    c.residents = w.residents([(f"blk.{i}.essai.weight", [0, 8, 0][i], [tailles[i] // 4, 1, 1, 1], 1 + i % 2,
                                c.donnees[i]) for i in range(3)])

    tables = []
    for couche in (1, 0):
        for j in range(3):
            for sorte, ctx in [(T.SORTE_CODES_CTX, 2), (T.SORTE_DELTA, 0), (T.SORTE_CODES_CTX, 0),
                               (T.SORTE_CODES_CTX, 1)]:
                f = np.zeros(256, np.int64)
                f[(couche + j + ctx) % 256] = 4000
                f[255] = 96
                if table_8 and sorte == T.SORTE_CODES_CTX:
                    f[255] = 95
                    f[0x08] = 1
                tables.append(T.Table.de(couche, j, sorte, ctx, f))
    tables.append(T.Table.de(1, 2, T.SORTE_COMPL_CTX, 17, np.full(16, 256)))
    tables.append(T.Table.de(0, 1, T.SORTE_CENTRES, 0, np.array([0.25, 1.4, 3.4, 6.0], np.float32)))
    c.tables = tables
    if not tables_apres:
        w.tables(tables)

    w.troncons(2, 3)
    c.repertoire, c.parties = [], []
    for couche in range(2):
        for x in range(3):
            flux = []
            for j in range(3):
                for s, n in [(T.SORTE_MEDIANES, 64), (T.SORTE_BIAIS, 256), (T.SORTE_DELTA, 160 + 16 * x),
                             (T.SORTE_CODES_CTX, 5000 + 37 * x)]:
                    o = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
                    flux.append((s, j, 0 if s == T.SORTE_DELTA else T.CONTEXTE_AUCUN, len(o), o))
            p, utiles = T.assembler_partie(couche, x, 0, 3, flux)
            en = w.partie(couche, x, p, empreinte_origine=int(rng.integers(1, 1 << 63)),
                          empreinte_canonique=int(rng.integers(1, 1 << 63)) if canonique else 0)
            assert en.utiles[0] == utiles and en.longueur[0] == p.size
            c.repertoire.append(en)
            c.parties.append(p)
    if tables_apres:
        w.tables(tables)
    if canonique:
        c.entete = T.Entete.type_(version=(1, 2), drapeaux=T.DRAPEAU_ALIGNE | T.DRAPEAU_CANONIQUE)
    else:
        c.entete = T.Entete.type_()
    c.entete.sha256_source[:] = [7] * 32
    c.entete.taille_source = 123_456_789
    c.taille = w.terminer(c.entete)
    return c


def _cle_table(t):
    return (t.couche, t.matrice, t.sorte, t.contexte)


@pytest.fixture(scope="module")
def fichier(tmp_path_factory):
    chemin = tmp_path_factory.mktemp("trc") / "aller_retour.trc"
    return chemin, _ecrire(chemin)


@pytest.mark.parametrize("tables_apres", [False, True])
def test_aller_retour_identique_181(tmp_path, tables_apres):
    chemin = tmp_path / "aller_retour.trc"
    c = _ecrire(chemin, tables_apres=tables_apres)
    f = T.Fichier.ouvrir(chemin)
    e = f.entete()
    attendu = c.entete.valeurs()
    lu = e.valeurs()
    attendu["sections"], attendu["taille_fichier"] = lu["sections"], chemin.stat().st_size
    assert lu == attendu
    assert e.taille_fichier % T.ALIGNEMENT == 0 and e.taille_fichier == c.taille
    assert f.meta() == c.meta_brute
    assert [p.cle for p in f.paires()] == ["general.architecture", "essai.couches_x", "jetons",
                                           "troncons.codeur.version"]
    assert f.paire("essai.couches_x").entier() == 2
    assert f.paire("jetons").valeur == ("tableau", 8, 2)
    assert f.paire("general.architecture").chaine() == "essai"
    assert f.paire("absente") is None
    assert [r.cle() for r in f.residents()] == [r.cle() for r in c.residents]
    octets = chemin.read_bytes()
    for r, d in zip(f.residents(), c.donnees):
        a = f.debut_donnees_residentes() + r.decalage
        assert octets[a:a + r.octets] == d
        assert r.decalage % 256 == 0 and T.empreinte64(d) == r.empreinte
        assert f.donnees_resident(r).tobytes() == d
    attendues = sorted(c.tables, key=_cle_table)
    assert [t.cle() for t in f.toutes_tables()] == [t.cle() for t in attendues]
    assert len(f.tables(1, 2)) == 5
    assert f.table(0, 1, T.SORTE_CENTRES, 0) is not None
    assert f.table(0, 1, T.SORTE_CENTRES, 1) is None
    assert [en.cle() for en in f.repertoire()] == [en.cle() for en in c.repertoire]
    for i, en in enumerate(f.repertoire()):
        p = np.frombuffer(octets[en.decalage:en.decalage + en.longueur[0]], np.uint8)
        assert (p == c.parties[i]).all()
        lue = T.lire_partie(p)
        assert (lue.couche, lue.expert, lue.niveau, lue.n_matrices) == (en.couche, en.expert, 0, 3)
        assert len(lue.flux) == 12 and lue.utiles == en.utiles[0]
        assert T.empreinte64(p[:lue.utiles]) == en.empreinte_niveau[0]
        for d in lue.flux:
            assert d.decalage % 16 == 0 and lue.octets_flux(d).size == d.produits
        assert (f.lire_partie(en.couche, en.expert) == p).all()
    # the opening reads the header, the resident table (not its data), TABLES and RÉPERTOIRE only
    s = e.sections
    assert f.octets_lus_a_l_ouverture() < s[T.SECTION_TRONCONS].longueur


def _fausse(source, tmp, nom, position, xor):
    b = bytearray(source.read_bytes())
    b[position] ^= xor
    c = tmp / nom
    c.write_bytes(bytes(b))
    return lambda: T.Fichier.ouvrir(c)


def _reempreinte(b, debut, fin):
    """Recomputes the fingerprint stored in b[fin-8:fin] over b[debut:fin-8]."""
    b[fin - 8:fin] = T.empreinte64(bytes(b[debut:fin - 8])).to_bytes(8, "little")


def _entete_change(source, tmp, nom, f):
    b = bytearray(source.read_bytes())
    h = b[:4096]
    f(h)
    b[:4096] = h
    _reempreinte(b, 0, 4096)
    c = tmp / nom
    c.write_bytes(bytes(b))
    return lambda: T.Fichier.ouvrir(c)


def test_cassures_refusees_238(fichier, tmp_path):
    chemin, _c = fichier
    f = T.Fichier.ouvrir(chemin)
    s = f.entete().sections
    assert _classe(_fausse(chemin, tmp_path, "c1.trc", 0, 0x20)) == "Magie"
    for pos, nom in [(8, "version"), (300, "reserve"), (4090, "empreinte"), (136, "section"), (72, "couches")]:
        assert _classe(_fausse(chemin, tmp_path, f"c-{nom}.trc", pos, 0x01)) == "Empreinte", nom

    def v9(h):
        h[10] = 9
    with pytest.raises(ErreurFormat) as e:
        _entete_change(chemin, tmp_path, "c-version-9.trc", v9)()
    assert e.value.classe == "Version" and "1.9" in e.value.message

    def canon_v10(h):
        h[12] |= 8
    assert _classe(_entete_change(chemin, tmp_path, "c-canon.trc", canon_v10)) == "Drapeaux"
    for i in (T.SECTION_META, T.SECTION_RESIDENTS, T.SECTION_TABLES, T.SECTION_REPERTOIRE):
        with pytest.raises(ErreurFormat):
            _fausse(chemin, tmp_path, f"s-{i}.trc", s[i].decalage + 9, 0x10)()
    b = chemin.read_bytes()
    (tmp_path / "tronque.trc").write_bytes(b[:-4096])
    assert _classe(lambda: T.Fichier.ouvrir(tmp_path / "tronque.trc")) == "Champ"
    (tmp_path / "court.trc").write_bytes(b[:1000])
    assert _classe(lambda: T.Fichier.ouvrir(tmp_path / "court.trc")) == "Es"
    assert _classe(lambda: T.Fichier.ouvrir(tmp_path / "absent.trc")) == "Es"
    en = f.entree(1, 2)
    p = np.frombuffer(b[en.decalage:en.decalage + en.longueur[0]], np.uint8)
    T.lire_partie(p)
    for pos, val, classe in [(0, 0x55, "Champ"), (64, 0x05, "Sorte"), (67, 1, "Reserve"), (40, 1, "Reserve"),
                             (p.size - 1, 1, "Reserve"), (64 + 16 + 1, 3, "Champ")]:
        q = p.copy()
        q[pos] = val
        assert _classe(lambda: T.lire_partie(q)) == classe, pos
    # a descriptor whose stream runs past the useful bytes, or starts inside the previous one
    q = p.copy()
    q[64 + 8:64 + 12] = np.frombuffer(struct.pack("<I", 1 << 30), np.uint8)
    assert _classe(lambda: T.lire_partie(q)) == "Limites"
    q = p.copy()
    q[64 + 16 + 4:64 + 16 + 8] = q[64 + 4:64 + 8]
    assert _classe(lambda: T.lire_partie(q)) == "Limites"


def test_each_refusal_class_is_reached(fichier, tmp_path):
    """One targeted, re-hashed change per check of the opening, so the check itself (not the
    fingerprint before it) must refuse, with its own class."""
    chemin, _c = fichier
    f = T.Fichier.ouvrir(chemin)
    s = [(x.decalage, x.longueur) for x in f.entete().sections]
    original = chemin.read_bytes()

    def avec(nom, changer, section=None):
        b = bytearray(original)
        changer(b)
        if section is not None:
            d, n = s[section]
            _reempreinte(b, d, d + n)
        c = tmp_path / nom
        c.write_bytes(bytes(b))
        return _classe(lambda: T.Fichier.ouvrir(c))

    dt, nt = s[T.SECTION_TABLES]
    rec0 = dt + 8
    # TABLES: reserved count word, a reserved record word, an unknown kind, a bad payload type,
    # frequencies not summing to 4096, a layer beyond the header, a duplicated key
    assert avec("t-res.trc", lambda b: b.__setitem__(dt + 4, 1), T.SECTION_TABLES) == "Reserve"
    assert avec("t-res2.trc", lambda b: b.__setitem__(rec0 + 6, 1), T.SECTION_TABLES) == "Reserve"
    assert avec("t-sorte.trc", lambda b: b.__setitem__(rec0 + 3, 0x05), T.SECTION_TABLES) == "Sorte"
    assert avec("t-type.trc", lambda b: b.__setitem__(rec0 + 5, 4), T.SECTION_TABLES) == "Champ"
    assert avec("t-somme.trc", lambda b: b.__setitem__(rec0 + 8, b[rec0 + 8] ^ 1), T.SECTION_TABLES) == "Champ"
    assert avec("t-couche.trc", lambda b: b.__setitem__(rec0, 7), T.SECTION_TABLES) == "Champ"

    def doublon(b):  # record 1 (layer 1, matrix 0, DELTA) becomes a second (1, 0, CODES_CTX, 2)
        r1 = rec0 + 520
        b[r1 + 3], b[r1 + 4] = b[rec0 + 3], b[rec0 + 4]
    assert avec("t-doublon.trc", doublon, T.SECTION_TABLES) == "Champ"

    dr, nr = s[T.SECTION_REPERTOIRE]
    # RÉPERTOIRE: reserved bytes 52..56, an entry naming another expert, an entry past TRONÇONS
    assert avec("r-res.trc", lambda b: b.__setitem__(dr + 52, 1), T.SECTION_REPERTOIRE) == "Reserve"
    assert avec("r-id.trc", lambda b: b.__setitem__(dr + 64 + 50, 2), T.SECTION_REPERTOIRE) == "Champ"
    assert avec("r-hors.trc", lambda b: b.__setitem__(dr + 7, 0x7F), T.SECTION_REPERTOIRE) == "Limites"
    assert avec("r-canon.trc", lambda b: b.__setitem__(dr + 56, 1), T.SECTION_REPERTOIRE) == "Limites"

    dm, nm = s[T.SECTION_META]
    # MÉTA: a value type beyond 12, a truncated pair (count one too high)
    cle0 = len("general.architecture")
    assert avec("m-type.trc", lambda b: b.__setitem__(dm + 16 + cle0, 13), T.SECTION_META) == "Champ"
    assert avec("m-n.trc", lambda b: b.__setitem__(dm, 5), T.SECTION_META) == "Limites"

    dres, nres = s[T.SECTION_RESIDENTS]
    # RÉSIDENTS: table fingerprint, padding after the table, an offset not on 256, zero dimensions
    assert avec("res-emp.trc", lambda b: b.__setitem__(dres + 8, b[dres + 8] ^ 1)) == "Empreinte"

    def res_change(off, val):
        def ch(b):
            b[dres + off] = val
            table = bytes(b[dres:dres + 8 + 128 * 3])
            b[dres + nres - 8:dres + nres] = T.empreinte64(table).to_bytes(8, "little")
        return ch
    assert avec("res-pad.trc", lambda b: b.__setitem__(dres + 8 + 128 * 3 + 5, 1)) == "Reserve"
    assert avec("res-nom.trc", res_change(8 + 60, 0x41)) == "Reserve"
    assert avec("res-dec.trc", res_change(8 + 128 + 104, 1)) == "Champ"
    assert avec("res-dims.trc", res_change(8 + 68, 0)) == "Champ"

    # header: overlapping sections, a section beyond the end, reserved sections 5-7, k > E,
    # matrices = 0, levels = 2 without the flag, alignment field
    def sect(i, champ, v):
        def ch(h):
            h[136 + 16 * i + 8 * champ:144 + 16 * i + 8 * champ] = v.to_bytes(8, "little")
        return ch
    assert _classe(_entete_change(chemin, tmp_path, "h-chev.trc", sect(T.SECTION_TABLES, 0, s[T.SECTION_META][0]))) \
        == "Limites"
    assert _classe(_entete_change(chemin, tmp_path, "h-fin.trc", sect(T.SECTION_TRONCONS, 1, 1 << 40))) == "Limites"
    assert _classe(_entete_change(chemin, tmp_path, "h-s5.trc", sect(5, 1, 1))) == "Reserve"
    assert _classe(_entete_change(chemin, tmp_path, "h-k.trc", lambda h: h.__setitem__(76, 9))) == "Champ"
    assert _classe(_entete_change(chemin, tmp_path, "h-m.trc", lambda h: h.__setitem__(78, 0))) == "Champ"
    assert _classe(_entete_change(chemin, tmp_path, "h-niv.trc", lambda h: h.__setitem__(121, 2))) == "Drapeaux"
    assert _classe(_entete_change(chemin, tmp_path, "h-al.trc", lambda h: h.__setitem__(17, 0x20))) == "Champ"
    assert _classe(_entete_change(chemin, tmp_path, "h-dim.trc", lambda h: h.__setitem__(80 + 12, 1))) == "Reserve"
    assert _classe(_entete_change(chemin, tmp_path, "h-ali.trc", sect(0, 0, 4096 + 16))) == "Champ"


def test_parts_read_back_checked(fichier, tmp_path):
    """verifier_partie and the read path: a changed useful byte is a fingerprint refusal, a part
    presented as another expert's is refused, reading into a torch host tensor works."""
    import torch
    chemin, c = fichier
    f = T.Fichier.ouvrir(chemin)
    en = f.entree(0, 1)
    p = f.lire_partie(0, 1)
    f.verifier_partie(0, 1, 0, p)
    q = p.copy()
    q[100] ^= 1
    assert _classe(lambda: f.verifier_partie(0, 1, 0, q)) == "Empreinte"
    assert _classe(lambda: f.verifier_partie(0, 2, 0, f.lire_partie(0, 2)[: en.utiles[0] - 1])) == "Limites"
    t = torch.zeros(en.longueur[0], dtype=torch.uint8)
    assert f.lire_partie(0, 1, dst=t) == en.longueur[0]
    assert (t.numpy() == p).all()
    b = bytearray(chemin.read_bytes())
    b[en.decalage + 200] ^= 1
    (tmp_path / "p.trc").write_bytes(bytes(b))
    g = T.Fichier.ouvrir(tmp_path / "p.trc")  # parts are not read at opening
    assert _classe(lambda: g.lire_partie(0, 1)) == "Empreinte"
    assert (g.lire_partie(0, 1, verifier=False) == np.frombuffer(bytes(b[en.decalage:en.decalage + en.longueur[0]]),
                                                                 np.uint8)).all()


def test_aller_retour_v12_canonique_303(tmp_path):
    chemin = tmp_path / "canonique.trc"
    c = _ecrire(chemin, canonique=True)
    f = T.Fichier.ouvrir(chemin)
    e = f.entete()
    assert e.version == (1, 2) and e.est_canonique() and not e.est_brut()
    assert [x.cle() for x in f.repertoire()] == [x.cle() for x in c.repertoire]
    for en in f.repertoire():
        assert en.empreinte_canonique != 0
        assert en.empreinte_du_decode(True) == en.empreinte_canonique
        assert en.empreinte_du_decode(False) == en.empreinte_origine
    b = chemin.read_bytes()
    d = e.sections[T.SECTION_REPERTOIRE].decalage
    assert int.from_bytes(b[d + 56:d + 64], "little") == c.repertoire[0].empreinte_canonique
    chemin0 = tmp_path / "non-canonique.trc"
    c0 = _ecrire(chemin0)
    f0 = T.Fichier.ouvrir(chemin0)
    assert not f0.entete().est_canonique()
    assert all(x.empreinte_canonique == 0 for x in f0.repertoire())
    assert f0.repertoire()[0].empreinte_du_decode(False) == c0.repertoire[0].empreinte_origine


def test_cassures_v12_refusees_329(tmp_path):
    chemin = tmp_path / "canonique-cassures.trc"
    _ecrire(chemin, canonique=True)
    T.Fichier.ouvrir(chemin)
    assert _classe(_entete_change(chemin, tmp_path, "v12-sous-11.trc", lambda h: h.__setitem__(10, 1))) == "Drapeaux"
    assert _classe(_entete_change(chemin, tmp_path, "v12-brut.trc",
                                  lambda h: h.__setitem__(12, h[12] | T.DRAPEAU_BRUT))) == "Drapeaux"
    assert _classe(_entete_change(chemin, tmp_path, "v12-bit4.trc", lambda h: h.__setitem__(12, h[12] | 16))) \
        == "Drapeaux"
    with pytest.raises(ErreurFormat) as e:
        _entete_change(chemin, tmp_path, "v13.trc", lambda h: h.__setitem__(10, 3))()
    assert e.value.classe == "Version" and "1.3" in e.value.message
    assert _classe(_entete_change(chemin, tmp_path, "v12-sans-drapeau.trc",
                                  lambda h: h.__setitem__(12, h[12] & ~T.DRAPEAU_CANONIQUE))) == "Limites"
    c8 = tmp_path / "canonique-table-8.trc"
    _ecrire(c8, canonique=True, table_8=True)
    assert _classe(lambda: T.Fichier.ouvrir(c8)) == "Champ"
    c80 = tmp_path / "v10-table-8.trc"
    _ecrire(c80, canonique=False, table_8=True)
    T.Fichier.ouvrir(c80)


def test_drapeau_rapide_v12_376(tmp_path):
    chemin = tmp_path / "rapide-base.trc"
    _ecrire(chemin)

    def rapide(h, plus=0):
        h[10] = 2
        h[12] |= T.DRAPEAU_RAPIDE | plus
    f = _entete_change(chemin, tmp_path, "rapide-ok.trc", rapide)()
    assert f.entete().est_rapide()
    assert _classe(_entete_change(chemin, tmp_path, "rapide-10.trc",
                                  lambda h: h.__setitem__(12, h[12] | T.DRAPEAU_RAPIDE))) == "Drapeaux"
    assert _classe(_entete_change(chemin, tmp_path, "rapide-brut.trc", lambda h: rapide(h, T.DRAPEAU_BRUT))) \
        == "Drapeaux"
    assert _classe(_entete_change(chemin, tmp_path, "rapide-canon.trc", lambda h: rapide(h, T.DRAPEAU_CANONIQUE))) \
        == "Drapeaux"


def test_temoin_du_temoin_403(fichier):
    _chemin, c = fichier
    p = c.parties[3].copy()
    assert (p == c.parties[3]).all()
    p[100] ^= 1
    assert not (p == c.parties[3]).all()
    assert T.empreinte64(p[:c.repertoire[3].utiles[0]]) != c.repertoire[3].empreinte_niveau[0]


def test_two_level_parts(tmp_path):
    """A v1.1 two-level file: level 1 ("TRC1") right after level 0, read in one request."""
    rng = np.random.default_rng(3)
    w = T.Ecrivain(tmp_path / "niveaux.trc")
    w.meta(b"", 0)
    w.residents([])
    w.tables([])
    w.troncons(1, 2)
    for x in range(2):
        f0 = [(T.SORTE_CODES_CTX, 0, T.CONTEXTE_AUCUN, 100, rng.integers(0, 256, 100, dtype=np.uint8))]
        f1 = [(T.SORTE_COMPL_CTX, 0, T.CONTEXTE_AUCUN, 50, rng.integers(0, 256, 5000, dtype=np.uint8))]
        p0, _ = T.assembler_partie(0, x, 0, 1, f0)
        p1, _ = T.assembler_partie(0, x, 1, 1, f1)
        with pytest.raises(T.ErreurUsage):
            w.partie(0, x, p1)  # a level-1 part given as level 0
        w.partie(0, x, p0, p1)
    e = T.Entete.type_(couches=1, experts=2, k=1, matrices=1, lignes=(64,), colonnes=(64,), version=(1, 1),
                       drapeaux=T.DRAPEAU_ALIGNE | T.DRAPEAU_NIVEAUX, niveaux=2)
    w.terminer(e)
    f = T.Fichier.ouvrir(tmp_path / "niveaux.trc")
    en = f.entree(0, 1)
    assert en.longueur[0] == 4096 and en.longueur[1] == 8192
    both = f.lire_partie(0, 1, niveaux=2)
    assert both.size == 3 * 4096
    assert T.lire_partie(both[4096:]).niveau == 1
    assert (f.lire_partie(0, 1, niveaux=1) == both[:4096]).all()


def test_writer_refuses_misuse(tmp_path):
    w = T.Ecrivain(tmp_path / "mal.trc")
    with pytest.raises(T.ErreurUsage):
        w.tables([])  # before MÉTA
    with pytest.raises(T.ErreurUsage):
        w.meta(T.paire_chaine("a", "b"), 2)  # two pairs announced, one given
    w.meta(T.paire_chaine("a", "b"), 1)
    with pytest.raises(T.ErreurUsage):
        w.residents([("x" * 65, 0, [1], 1, b"1234")])
    w.residents([])
    w.troncons(1, 2)
    p, _ = T.assembler_partie(0, 0, 0, 1, [(T.SORTE_DELTA, 0, 0, 4, b"abcd")])
    w.partie(0, 0, p)
    with pytest.raises(T.ErreurUsage):
        w.partie(0, 0, p)  # twice
    with pytest.raises(T.ErreurUsage):
        w.partie(0, 1, p)  # the part names expert 0
    w.tables([])
    with pytest.raises(T.ErreurUsage):
        w.terminer(T.Entete.type_(couches=1, experts=2, k=1, matrices=1, lignes=(64,), colonnes=(64,)))  # (0, 1) missing


# ------------------------------------------------------------------ the synthetic model file

def _blocs_vers_octets(blocs, biais, canonique):
    out = []
    for j in range(3):
        b = np.asarray(blocs[j], np.uint8).reshape(-1, 17).copy()
        if canonique:
            q = b[:, 1:]
            lo, hi = q & 15, q >> 4
            lo[lo == 8] = 0
            hi[hi == 8] = 0
            b[:, 1:] = lo | (hi << 4)
        out.append(b.tobytes())
    return b"".join(out) + b"".join(np.asarray(biais[j], np.float32).tobytes() for j in range(3))


def test_synthetic_model_file(tmp_path):
    """trc_synth_fichier: tables and parts equal to the encoder's; fingerprints equal hashlib over
    the generated experts (as generated, and canonical); routers equal the generator; the oracle's
    decode of every part read back from disk hashes to the directory's canonical fingerprint."""
    dims = DimsExpert.de([64, 64, 96], [96, 96, 64])
    chemin = tmp_path / "synth.trc"
    taille = T.synth_fichier(chemin, 42, 2, 4, 2, dims, N_delta=4, N_codes=8, n_fils=4)
    assert taille == chemin.stat().st_size
    f = T.Fichier.ouvrir(chemin)
    e = f.entete()
    assert (e.version, e.couches, e.experts, e.k, e.matrices, e.niveaux) == ((1, 2), 2, 4, 2, 3, 1)
    assert e.est_canonique() and list(e.lignes[:3]) == [64, 64, 96] and list(e.colonnes[:3]) == [96, 96, 64]
    assert f.paire("gpt-oss.expert_count").entier() == 4
    assert f.paire("troncons.synth.graine").entier() == 42
    assert bytes(e.sha256_source) == hashlib.sha256(f.meta()[8:]).digest()
    assert e.sections[T.SECTION_TABLES].decalage > e.sections[T.SECTION_TRONCONS].decalage
    res = f.residents()
    assert [r.nom for r in res] == ["blk.0.ffn_gate_inp.weight", "blk.1.ffn_gate_inp.weight"]
    for c in range(2):
        couche = codeur.CoucheSynthetique(42, c, 4, dims, N_delta=4, N_codes=8, n_fils=4)
        assert (f.freqs_couche(c) == couche.freqs()).all()
        r = np.stack([codeur.synth_normale_bf16(42 + c, 3, x, 96, 0.02) for x in range(4)])
        assert (f.donnees_resident(res[c]).view(np.uint16) == (r.view(np.uint32) >> 16).astype(np.uint16).ravel()).all()
        luts = O.luts_couche(f.freqs_couche(c))
        for x in range(4):
            en = f.entree(c, x)
            p = f.lire_partie(c, x)
            assert (p == couche.partie(x)).all() and en.utiles[0] == couche.utiles(x)
            bl, bi = codeur.synth_expert(42, c, x, dims)
            h0 = hashlib.sha256(_blocs_vers_octets(bl, bi, False)).digest()
            h1 = hashlib.sha256(_blocs_vers_octets(bl, bi, True)).digest()
            assert en.empreinte_origine == int.from_bytes(h0[:8], "little")
            assert en.empreinte_canonique == int.from_bytes(h1[:8], "little")
            assert T.empreinte_expert(bl, bi, dims) == en.empreinte_origine
            empl, ctl = O.decoder_expert(p.tobytes(), luts, list(dims.lignes), list(dims.colonnes))
            assert (ctl == 0).all()
            assert T.empreinte_emplacement(empl, dims) == en.empreinte_canonique
        couche.liberer()
