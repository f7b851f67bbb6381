"""Host mirror of the .trc v1.2 container (the Rust crate ``trc_format``,
moteur/crates/trc-format/src/lib.rs and src/meta.rs), over the C-ABI of libtroncons_hip.so
(csrc/conteneur.cpp, csrc/empreinte.hpp).

Same names and meaning as the reference: ``Fichier.ouvrir`` reads and checks the header, MÉTA, the
resident table, TABLES and RÉPERTOIRE, and refuses a damaged file with ``ErreurFormat`` whose
``classe`` is the reference's variant (Es, Magie, Version, Drapeaux, Sorte, Champ, Empreinte,
Reserve, Limites); ``lire_partie`` checks one part; ``Ecrivain`` writes a file section by section;
``empreinte64`` is the first 8 bytes of SHA-256, little-endian. Parts are read with pread straight
into the caller's buffer (a pinned host tensor for the streaming path).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from .noyaux import DimsExpert, ErreurUsage, _statut, bibliotheque

# ---------------------------------------------------------------------------------- constants

MAGIE = b"TRONCONS"
ALIGNEMENT = 4096
TAILLE_ENTETE = 4096
VERSION_MAJEURE, VERSION_MINEURE = 1, 2

DRAPEAU_ALIGNE, DRAPEAU_NIVEAUX, DRAPEAU_BRUT, DRAPEAU_CANONIQUE, DRAPEAU_RAPIDE = 1, 2, 4, 8, 32

SECTION_META, SECTION_RESIDENTS, SECTION_TABLES, SECTION_REPERTOIRE, SECTION_TRONCONS = range(5)

SORTE_MEDIANES, SORTE_BIAIS, SORTE_DELTA, SORTE_CODES_CTX = 0x01, 0x02, 0x03, 0x04
SORTE_CODES_BRUTS, SORTE_ECHELLES_BRUTES = 0x06, 0x07
SORTE_BASE_CTX, SORTE_COMPL_CTX, SORTE_CENTRES = 0x10, 0x11, 0x12
CONTEXTE_AUCUN = 0xFF

TAILLE_ENTREE_REPERTOIRE = 64
TAILLE_ENTREE_RESIDENT = 128

_CLASSES = {16: "Es", 17: "Magie", 18: "Version", 19: "Drapeaux", 20: "Sorte", 21: "Champ", 22: "Empreinte",
            23: "Reserve", 24: "Limites"}


class ErreurFormat(RuntimeError):
    """ErreurFormat (trc-format/src/lib.rs:129-148); ``classe`` names the variant."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{_CLASSES.get(code, code)} : {message}")
        self.code = code
        self.classe = _CLASSES.get(code, str(code))
        self.message = message


def _verifier(r: int) -> None:
    if r in _CLASSES:
        raise ErreurFormat(r, bibliotheque().trc_derniere_erreur().decode("utf-8", "replace"))
    _statut(r)


def canoniser_demi(c: int) -> int:
    """canoniser_demi (trc-format/src/lib.rs:69-73): nibble 8 (-0) becomes 0."""
    return 0 if c == 8 else c


def canoniser_octet(o: int) -> int:
    """canoniser_octet (lib.rs:75-79)"""
    return canoniser_demi(o & 15) | (canoniser_demi(o >> 4) << 4)


def porte_un_8(o: int) -> bool:
    """porte_un_8 (lib.rs:81-84): the byte carries a nibble 8."""
    return (o & 15) == 8 or (o >> 4) == 8


# ------------------------------------------------------------------------------- structures

class Section(C.Structure):
    _fields_ = [("decalage", C.c_uint64), ("longueur", C.c_uint64)]

    def fin(self) -> int:
        return self.decalage + self.longueur


class Entete(C.Structure):
    """Entete (lib.rs:250-272)"""
    _fields_ = [("version_majeure", C.c_uint16), ("version_mineure", C.c_uint16), ("drapeaux", C.c_uint32),
                ("taille_fichier", C.c_uint64), ("sha256_source", C.c_uint8 * 32), ("taille_source", C.c_uint64),
                ("couches", C.c_uint16), ("experts", C.c_uint16), ("k", C.c_uint16), ("matrices", C.c_uint16),
                ("lignes", C.c_uint32 * 4), ("colonnes", C.c_uint32 * 4), ("poids_par_bloc", C.c_uint32),
                ("octets_par_bloc", C.c_uint32), ("type_ggml", C.c_uint8), ("niveaux", C.c_uint8),
                ("classes_echelle", C.c_uint8), ("reserve0", C.c_uint8), ("partition", C.c_uint8 * 8),
                ("reserve1", C.c_uint32), ("sections", Section * 8)]

    @property
    def version(self):
        return (self.version_majeure, self.version_mineure)

    def est_brut(self) -> bool:
        return bool(self.drapeaux & DRAPEAU_BRUT)

    def est_rapide(self) -> bool:
        return bool(self.drapeaux & DRAPEAU_RAPIDE)

    def est_canonique(self) -> bool:
        return bool(self.drapeaux & DRAPEAU_CANONIQUE)

    def valeurs(self) -> dict:
        """Every field as plain Python values (for comparisons)."""
        d = {}
        for nom, _t in self._fields_:
            v = getattr(self, nom)
            if nom == "sections":
                v = [(s.decalage, s.longueur) for s in v]
            elif isinstance(v, C.Array):
                v = list(v)
            d[nom] = v
        return d

    @classmethod
    def type_(cls, couches=2, experts=3, k=2, matrices=3, lignes=(64, 64, 32), colonnes=(64, 64, 64), version=(1, 0),
              drapeaux=DRAPEAU_ALIGNE, niveaux=1) -> "Entete":
        e = cls()
        e.version_majeure, e.version_mineure = version
        e.drapeaux = drapeaux
        e.couches, e.experts, e.k, e.matrices = couches, experts, k, matrices
        for j in range(len(lignes)):
            e.lignes[j], e.colonnes[j] = lignes[j], colonnes[j]
        e.poids_par_bloc, e.octets_par_bloc, e.type_ggml = 32, 17, 39
        e.niveaux, e.classes_echelle = niveaux, 3
        return e


class EntreeRepertoire(C.Structure):
    """EntreeRepertoire (lib.rs:444-500), the 64 on-disk bytes."""
    _fields_ = [("decalage", C.c_uint64), ("longueur", C.c_uint32 * 2), ("utiles", C.c_uint32 * 2),
                ("empreinte_origine", C.c_uint64), ("empreinte_niveau", C.c_uint64 * 2), ("couche", C.c_uint16),
                ("expert", C.c_uint16), ("reserve", C.c_uint32), ("empreinte_canonique", C.c_uint64)]

    def empreinte_du_decode(self, canonique: bool) -> int:
        return self.empreinte_canonique if canonique else self.empreinte_origine

    def longueur_jusqua(self, niveaux: int) -> int:
        return sum(self.longueur[:niveaux])

    def cle(self):
        return (self.decalage, tuple(self.longueur), tuple(self.utiles), self.empreinte_origine,
                tuple(self.empreinte_niveau), self.couche, self.expert, self.empreinte_canonique)


class Resident(C.Structure):
    """TenseurResident (lib.rs:683-693), the 128 on-disk bytes."""
    _fields_ = [("nom_", C.c_char * 64), ("type_ggml", C.c_uint32), ("n_dims", C.c_uint32), ("ne", C.c_uint64 * 4),
                ("decalage", C.c_uint64), ("octets", C.c_uint64), ("empreinte", C.c_uint64)]

    @property
    def nom(self) -> str:
        return bytes(self)[:64].rstrip(b"\0").decode("utf-8")

    def cle(self):
        return (self.nom, self.type_ggml, self.n_dims, tuple(self.ne), self.decalage, self.octets, self.empreinte)


class _Charge(C.Union):
    _fields_ = [("frequences", C.c_uint16 * 256), ("centres", C.c_float * 4)]


class Table(C.Structure):
    """Table (lib.rs:554-560) with its Charge (lib.rs:518-551)."""
    _fields_ = [("couche", C.c_uint16), ("matrice", C.c_uint8), ("sorte", C.c_uint8), ("contexte", C.c_uint8),
                ("type_charge", C.c_uint8), ("reserve", C.c_uint16), ("charge", _Charge)]

    @classmethod
    def de(cls, couche, matrice, sorte, contexte, charge) -> "Table":
        """charge: 16 or 256 frequencies (types 1, 2) or 4 float centres (type 3, a tuple of floats)."""
        t = cls()
        t.couche, t.matrice, t.sorte, t.contexte = couche, matrice, sorte, contexte
        a = np.asarray(charge)
        if a.dtype.kind == "f":
            t.type_charge = 3
            for i in range(4):
                t.charge.centres[i] = float(a[i])
        else:
            t.type_charge = 1 if a.size == 16 else 2
            for i, v in enumerate(a.astype(np.int64)):
                t.charge.frequences[i] = int(v)
        return t

    def frequences(self):
        if self.type_charge == 1:
            return np.array(self.charge.frequences[:16], np.uint16)
        if self.type_charge == 2:
            return np.array(self.charge.frequences[:], np.uint16)
        return None

    def centres(self):
        return np.array(self.charge.centres[:], np.float32) if self.type_charge == 3 else None

    def cle(self):
        payload = (tuple(self.frequences()) if self.type_charge != 3 else tuple(self.centres()))
        return (self.couche, self.matrice, self.sorte, self.contexte, self.type_charge, payload)


class _PaireMeta(C.Structure):
    _fields_ = [("debut", C.c_uint64), ("fin", C.c_uint64), ("cle", C.c_uint64), ("lg_cle", C.c_uint64),
                ("type", C.c_uint32), ("type_elem", C.c_uint32), ("n", C.c_uint64), ("chaine", C.c_uint64),
                ("u", C.c_uint64), ("i", C.c_int64), ("f", C.c_double)]


class DescFlux(C.Structure):
    """DescFlux (lib.rs:780-787), the 16 on-disk bytes."""
    _fields_ = [("sorte", C.c_uint8), ("matrice", C.c_uint8), ("contexte", C.c_uint8), ("reserve", C.c_uint8),
                ("decalage", C.c_uint32), ("longueur", C.c_uint32), ("produits", C.c_uint32)]


class _PartieInfo(C.Structure):
    _fields_ = [("couche", C.c_uint16), ("expert", C.c_uint16), ("niveau", C.c_uint8), ("n_matrices", C.c_uint8),
                ("n_flux", C.c_uint16), ("utiles", C.c_uint32)]


class _FluxAEcrire(C.Structure):
    _fields_ = [("sorte", C.c_uint8), ("matrice", C.c_uint8), ("contexte", C.c_uint8), ("reserve", C.c_uint8),
                ("produits", C.c_uint32), ("octets", C.c_void_p), ("longueur", C.c_uint64)]


# ------------------------------------------------------------------------------ declarations

_u8p = C.POINTER(C.c_uint8)


def _declarer(l):
    if getattr(l, "_trc_conteneur", False):
        return l
    l.trc_empreinte64.argtypes = [C.c_void_p, C.c_uint64]
    l.trc_empreinte64.restype = C.c_uint64
    l.trc_sha256.argtypes = [C.c_void_p, C.c_uint64, C.c_void_p]
    l.trc_empreinte_expert.argtypes = [C.POINTER(C.c_void_p), C.POINTER(C.c_void_p), C.POINTER(DimsExpert)]
    l.trc_empreinte_expert.restype = C.c_uint64
    l.trc_empreinte_emplacement.argtypes = [C.c_void_p, C.POINTER(DimsExpert)]
    l.trc_empreinte_emplacement.restype = C.c_uint64
    l.trc_partie_lire.argtypes = [C.c_void_p, C.c_uint64, C.POINTER(_PartieInfo)]
    l.trc_fichier_ouvrir.argtypes = [C.c_char_p, C.POINTER(C.c_void_p)]
    l.trc_fichier_fermer.argtypes = [C.c_void_p]
    l.trc_fichier_entete.argtypes = [C.c_void_p]
    l.trc_fichier_entete.restype = C.POINTER(Entete)
    l.trc_fichier_meta.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
    l.trc_fichier_meta.restype = C.c_uint64
    l.trc_fichier_n_paires.argtypes = [C.c_void_p]
    l.trc_fichier_n_paires.restype = C.c_uint64
    l.trc_fichier_paires.argtypes = [C.c_void_p]
    l.trc_fichier_paires.restype = C.POINTER(_PaireMeta)
    l.trc_fichier_chercher_paire.argtypes = [C.c_void_p, C.c_char_p]
    l.trc_fichier_chercher_paire.restype = C.c_int64
    l.trc_fichier_n_residents.argtypes = [C.c_void_p]
    l.trc_fichier_n_residents.restype = C.c_uint32
    l.trc_fichier_residents.argtypes = [C.c_void_p]
    l.trc_fichier_residents.restype = C.POINTER(Resident)
    l.trc_fichier_debut_donnees.argtypes = [C.c_void_p]
    l.trc_fichier_debut_donnees.restype = C.c_uint64
    l.trc_fichier_n_tables.argtypes = [C.c_void_p]
    l.trc_fichier_n_tables.restype = C.c_uint32
    l.trc_fichier_tables.argtypes = [C.c_void_p]
    l.trc_fichier_tables.restype = C.POINTER(Table)
    l.trc_fichier_table.argtypes = [C.c_void_p, C.c_uint16, C.c_uint8, C.c_uint8, C.c_uint8]
    l.trc_fichier_table.restype = C.POINTER(Table)
    l.trc_fichier_freqs_couche.argtypes = [C.c_void_p, C.c_uint16, C.c_void_p]
    l.trc_fichier_repertoire.argtypes = [C.c_void_p]
    l.trc_fichier_repertoire.restype = C.POINTER(EntreeRepertoire)
    l.trc_fichier_entree.argtypes = [C.c_void_p, C.c_uint16, C.c_uint16]
    l.trc_fichier_entree.restype = C.POINTER(EntreeRepertoire)
    l.trc_fichier_octets_lus.argtypes = [C.c_void_p]
    l.trc_fichier_octets_lus.restype = C.c_uint64
    l.trc_fichier_lire.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.c_void_p]
    l.trc_fichier_lire_partie.argtypes = [C.c_void_p, C.c_uint16, C.c_uint16, C.c_uint32, C.c_void_p, C.c_uint64,
                                          C.c_int, C.POINTER(C.c_uint64)]
    l.trc_fichier_verifier_partie.argtypes = [C.c_void_p, C.c_uint16, C.c_uint16, C.c_uint32, C.c_void_p,
                                              C.c_uint64]
    l.trc_ecrivain_creer.argtypes = [C.c_char_p]
    l.trc_ecrivain_creer.restype = C.c_void_p
    l.trc_ecrivain_abandonner.argtypes = [C.c_void_p]
    l.trc_ecrivain_meta.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64]
    l.trc_ecrivain_residents.argtypes = [C.c_void_p, C.POINTER(Resident), C.POINTER(C.c_void_p), C.c_uint32]
    l.trc_ecrivain_tables.argtypes = [C.c_void_p, C.POINTER(Table), C.c_uint32]
    l.trc_ecrivain_troncons.argtypes = [C.c_void_p, C.c_uint16, C.c_uint16]
    l.trc_ecrivain_partie.argtypes = [C.c_void_p, C.c_uint16, C.c_uint16, C.c_void_p, C.c_uint64, C.c_void_p,
                                      C.c_uint64, C.c_uint64, C.c_uint64, C.POINTER(EntreeRepertoire)]
    l.trc_ecrivain_terminer.argtypes = [C.c_void_p, C.POINTER(Entete), C.POINTER(C.c_uint64)]
    l.trc_assembler_partie.argtypes = [C.c_uint16, C.c_uint16, C.c_uint8, C.c_uint8, C.POINTER(_FluxAEcrire),
                                       C.c_uint32, C.c_void_p, C.c_uint64, C.POINTER(C.c_uint32)]
    l.trc_assembler_partie.restype = C.c_uint64
    l.trc_synth_fichier.argtypes = [C.c_char_p, C.c_uint64, C.c_uint16, C.c_uint16, C.c_uint16,
                                    C.POINTER(DimsExpert), C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint64)]
    l._trc_conteneur = True
    return l


def _l():
    return _declarer(bibliotheque())


def _octets(o) -> np.ndarray:
    """A contiguous uint8 numpy view of bytes / bytearray / numpy data."""
    if isinstance(o, np.ndarray):
        return np.ascontiguousarray(o).view(np.uint8).reshape(-1)
    return np.frombuffer(bytes(o), np.uint8)


def _chemin(chemin) -> bytes:
    return str(chemin).encode()


# ---------------------------------------------------------------------------------- functions

def empreinte64(octets) -> int:
    """empreinte64 (lib.rs:111-114)"""
    a = _octets(octets)
    return int(_l().trc_empreinte64(a.ctypes.data, a.size))


def empreinte64_morceaux(morceaux) -> int:
    """empreinte64_morceaux (lib.rs:117-124)"""
    return empreinte64(b"".join(bytes(_octets(m)) for m in morceaux))


def sha256(octets) -> bytes:
    a = _octets(octets)
    out = (C.c_uint8 * 32)()
    _l().trc_sha256(a.ctypes.data, a.size, out)
    return bytes(out)


def empreinte_expert(blocs17, biais, dims: DimsExpert) -> int:
    """empreinte64 of an expert: its 17-byte blocks (j = 0, 1, 2), then its f32 biases."""
    bl = [np.ascontiguousarray(b, np.uint8) for b in blocs17]
    bi = [np.ascontiguousarray(b, np.float32) for b in biais]
    pb = (C.c_void_p * 3)(*[b.ctypes.data for b in bl])
    pi = (C.c_void_p * 3)(*[b.ctypes.data for b in bi])
    return int(_l().trc_empreinte_expert(pb, pi, C.byref(dims)))


def empreinte_emplacement(emplacement, dims: DimsExpert) -> int:
    """empreinte_emplacement (trc-ordo/src/lib.rs:238-262), from a decoded slot copied to the host."""
    a = _octets(emplacement)
    return int(_l().trc_empreinte_emplacement(a.ctypes.data, C.byref(dims)))


def paire_chaine(cle: str, valeur: str) -> bytes:
    """paire_chaine (meta.rs:163-171): one serialised GGUF string pair."""
    c, v = cle.encode(), valeur.encode()
    return len(c).to_bytes(8, "little") + c + (8).to_bytes(4, "little") + len(v).to_bytes(8, "little") + v


def serialiser_meta(paires_brutes: bytes, n_paires: int, ajouts=()) -> bytes:
    """serialiser_meta (lib.rs:915-926)"""
    b = (n_paires + len(ajouts)).to_bytes(8, "little") + paires_brutes + b"".join(ajouts)
    return b + empreinte64(b).to_bytes(8, "little")


@dataclass
class Partie:
    """Partie (lib.rs:790-811)"""
    couche: int
    expert: int
    niveau: int
    n_matrices: int
    utiles: int
    flux: list
    octets: np.ndarray

    def octets_flux(self, d: DescFlux) -> np.ndarray:
        return self.octets[d.decalage:d.decalage + d.longueur]

    def trouver(self, sorte: int, matrice: int):
        for d in self.flux:
            if d.sorte == sorte and d.matrice == matrice:
                return d
        return None


def lire_partie(octets) -> Partie:
    """lire_partie (lib.rs:813-866); raises ErreurFormat."""
    a = _octets(octets)
    info = _PartieInfo()
    _verifier(_l().trc_partie_lire(a.ctypes.data, a.size, C.byref(info)))
    flux = [DescFlux.from_buffer_copy(a[64 + 16 * i:80 + 16 * i].tobytes()) for i in range(info.n_flux)]
    return Partie(info.couche, info.expert, info.niveau, info.n_matrices, info.utiles, flux, a)


def assembler_partie(couche: int, expert: int, niveau: int, n_matrices: int, flux) -> tuple[np.ndarray, int]:
    """assembler_partie (lib.rs:879-910): flux = [(sorte, matrice, contexte, produits, octets)].
    Returns (the part, a multiple of 4 096 bytes; its useful bytes)."""
    arrs = [_octets(f[4]) for f in flux]
    fe = (_FluxAEcrire * max(1, len(flux)))()
    for i, (s, m, ctx, prod, _o) in enumerate(flux):
        fe[i].sorte, fe[i].matrice, fe[i].contexte, fe[i].produits = s, m, ctx, prod
        fe[i].octets, fe[i].longueur = arrs[i].ctypes.data, arrs[i].size
    u = C.c_uint32()
    n = _l().trc_assembler_partie(couche, expert, niveau, n_matrices, fe, len(flux), None, 0, C.byref(u))
    if n == 0:
        _statut(1)
    out = np.zeros(n, np.uint8)
    _l().trc_assembler_partie(couche, expert, niveau, n_matrices, fe, len(flux), out.ctypes.data, n, C.byref(u))
    return out, int(u.value)


def synth_fichier(chemin, graine: int, couches: int, experts: int, k: int, dims: DimsExpert, N_delta: int = 4,
                  N_codes: int = 16, n_fils: int = 8) -> int:
    """A synthetic model as a v1.2 CANONIQUE .trc file (role of bins/trc-codeur); returns its size."""
    t = C.c_uint64()
    _verifier(_l().trc_synth_fichier(_chemin(chemin), graine, couches, experts, k, C.byref(dims), N_delta, N_codes,
                                     n_fils, C.byref(t)))
    return int(t.value)


# ------------------------------------------------------------------------------------ reader

@dataclass
class PaireMeta:
    """PaireMeta (meta.rs:21-30); ``valeur`` is an int, float, bool, str, or ("tableau", type, n)."""
    cle: str
    type_gguf: int
    debut: int
    fin: int
    valeur: object

    def entier(self):
        return self.valeur if isinstance(self.valeur, int) and not isinstance(self.valeur, bool) and \
            self.valeur >= 0 else None

    def reel(self):
        return self.valeur if isinstance(self.valeur, float) else None

    def chaine(self):
        return self.valeur if isinstance(self.valeur, str) else None


class Fichier:
    """Fichier (lib.rs:930-1141): an opened, checked .trc file."""

    def __init__(self, poignee: int, chemin):
        self._p = C.c_void_p(poignee)
        self.chemin = chemin

    @classmethod
    def ouvrir(cls, chemin) -> "Fichier":
        p = C.c_void_p()
        _verifier(_l().trc_fichier_ouvrir(_chemin(chemin), C.byref(p)))
        return cls(p.value, chemin)

    def fermer(self) -> None:
        if self._p:
            _l().trc_fichier_fermer(self._p)
            self._p = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.fermer()

    def __del__(self):
        try:
            self.fermer()
        except Exception:
            pass

    def entete(self) -> Entete:
        return Entete.from_buffer_copy(_l().trc_fichier_entete(self._p).contents)

    def meta(self) -> bytes:
        """u64 n then the pairs, fingerprint excluded (lib.rs:1099-1101)."""
        p = C.c_void_p()
        n = _l().trc_fichier_meta(self._p, C.byref(p))
        return C.string_at(p, n)

    def paires(self) -> list:
        meta = self.meta()
        corps = meta[8:]
        n = _l().trc_fichier_n_paires(self._p)
        tab = _l().trc_fichier_paires(self._p)
        out = []
        for i in range(n):
            m = tab[i]
            cle = corps[m.cle:m.cle + m.lg_cle].decode("utf-8")
            if m.type == 9:
                v = ("tableau", m.type_elem, m.n)
            elif m.type == 8:
                v = corps[m.chaine:m.chaine + m.n].decode("utf-8")
            elif m.type == 7:
                v = bool(m.u)
            elif m.type in (0, 2, 4, 10):
                v = int(m.u)
            elif m.type in (1, 3, 5, 11):
                v = int(m.i)
            else:
                v = float(m.f)
            out.append(PaireMeta(cle, m.type, m.debut, m.fin, v))
        return out

    def paire(self, cle: str):
        i = _l().trc_fichier_chercher_paire(self._p, cle.encode())
        return None if i < 0 else self.paires()[i]

    def residents(self) -> list:
        n = _l().trc_fichier_n_residents(self._p)
        t = _l().trc_fichier_residents(self._p)
        return [Resident.from_buffer_copy(t[i]) for i in range(n)]

    def debut_donnees_residentes(self) -> int:
        return int(_l().trc_fichier_debut_donnees(self._p))

    def donnees_resident(self, r: Resident) -> np.ndarray:
        return self.lire(self.debut_donnees_residentes() + r.decalage, r.octets)

    def toutes_tables(self) -> list:
        n = _l().trc_fichier_n_tables(self._p)
        t = _l().trc_fichier_tables(self._p)
        return [Table.from_buffer_copy(t[i]) for i in range(n)]

    def tables(self, couche: int, matrice: int) -> list:
        return [t for t in self.toutes_tables() if t.couche == couche and t.matrice == matrice]

    def table(self, couche: int, matrice: int, sorte: int, contexte: int):
        p = _l().trc_fichier_table(self._p, couche, matrice, sorte, contexte)
        return Table.from_buffer_copy(p.contents) if p else None

    def freqs_couche(self, couche: int) -> np.ndarray:
        """u16[3][4][256]: DELTA ctx 0 and CODES_CTX ctx 0..2 of each matrix (trc-ordo/src/lib.rs:265-273)."""
        out = np.zeros((3, 4, 256), np.uint16)
        _verifier(_l().trc_fichier_freqs_couche(self._p, couche, out.ctypes.data))
        return out

    def repertoire(self) -> list:
        e = self.entete()
        t = _l().trc_fichier_repertoire(self._p)
        return [EntreeRepertoire.from_buffer_copy(t[i]) for i in range(e.couches * e.experts)]

    def entree(self, couche: int, expert: int) -> EntreeRepertoire:
        p = _l().trc_fichier_entree(self._p, couche, expert)
        if not p:
            raise ErreurUsage(f"({couche}, {expert}) hors du fichier")
        return EntreeRepertoire.from_buffer_copy(p.contents)

    def octets_lus_a_l_ouverture(self) -> int:
        return int(_l().trc_fichier_octets_lus(self._p))

    def lire(self, decalage: int, octets: int, dst=None) -> np.ndarray:
        out = np.empty(octets, np.uint8) if dst is None else dst
        adr = out.ctypes.data if isinstance(out, np.ndarray) else int(out.data_ptr())
        _verifier(_l().trc_fichier_lire(self._p, decalage, octets, adr))
        return out

    def lire_partie(self, couche: int, expert: int, niveaux: int = 1, verifier: bool = True, dst=None):
        """Levels 0..niveaux-1 in one read, checked (fingerprint, structure, identity) when
        ``verifier``. ``dst``: a numpy array or a host torch tensor (pinned for the streaming path)
        of at least longueur_jusqua(niveaux) bytes; returns the bytes read (or the new array)."""
        n = self.entree(couche, expert).longueur_jusqua(niveaux)
        out = np.empty(n, np.uint8) if dst is None else dst
        if isinstance(out, np.ndarray):
            adr, cap = out.ctypes.data, out.nbytes
        else:
            adr, cap = int(out.data_ptr()), out.numel() * out.element_size()
        lu = C.c_uint64()
        _verifier(_l().trc_fichier_lire_partie(self._p, couche, expert, niveaux, adr, cap, int(verifier), C.byref(lu)))
        return out if dst is None else int(lu.value)

    def verifier_partie(self, couche: int, expert: int, niveau: int, octets) -> None:
        """verifier_partie (trc-codec/src/lib.rs:264-275) with the identity checks of reconstruire."""
        a = _octets(octets)
        _verifier(_l().trc_fichier_verifier_partie(self._p, couche, expert, niveau, a.ctypes.data, a.size))


# ------------------------------------------------------------------------------------ writer

class Ecrivain:
    """Ecrivain (lib.rs:1149-1239): MÉTA, RÉSIDENTS, TABLES, TRONÇONS, one call per expert, then
    ``terminer``. TABLES may also come after the last part."""

    def __init__(self, chemin):
        self._p = _l().trc_ecrivain_creer(_chemin(chemin))
        if not self._p:
            raise ErreurFormat(16, _l().trc_derniere_erreur().decode("utf-8", "replace"))

    def meta(self, paires: bytes, n_paires: int) -> None:
        a = _octets(paires)
        _verifier(_l().trc_ecrivain_meta(self._p, a.ctypes.data if a.size else None, a.size, n_paires))

    def residents(self, tenseurs) -> list:
        """tenseurs = [(nom, type_ggml, ne, n_dims, octets)]; returns the entries as written."""
        n = len(tenseurs)
        rs = (Resident * max(1, n))()
        arrs = []
        for i, (nom, tg, ne, nd, o) in enumerate(tenseurs):
            b = nom.encode("utf-8")
            if len(b) > 64 or b"\0" in b:
                raise ErreurUsage(f"nom de tenseur resident {nom!r} : au plus 64 octets UTF-8 sans zero")
            C.memmove(C.addressof(rs[i]), b, len(b))
            rs[i].type_ggml, rs[i].n_dims = tg, nd
            for j in range(4):
                rs[i].ne[j] = ne[j] if j < len(ne) else 1
            a = _octets(o)
            arrs.append(a)
            rs[i].octets = a.size
        ptrs = (C.c_void_p * max(1, n))(*[a.ctypes.data for a in arrs])
        _verifier(_l().trc_ecrivain_residents(self._p, rs, ptrs, n))
        return [Resident.from_buffer_copy(rs[i]) for i in range(n)]

    def tables(self, tables) -> None:
        arr = (Table * max(1, len(tables)))(*tables)
        _verifier(_l().trc_ecrivain_tables(self._p, arr, len(tables)))

    def troncons(self, couches: int, experts: int) -> None:
        _verifier(_l().trc_ecrivain_troncons(self._p, couches, experts))

    def partie(self, couche: int, expert: int, niveau0, niveau1=None, empreinte_origine: int = 0,
               empreinte_canonique: int = 0) -> EntreeRepertoire:
        a0 = _octets(niveau0)
        a1 = None if niveau1 is None else _octets(niveau1)
        en = EntreeRepertoire()
        _verifier(_l().trc_ecrivain_partie(self._p, couche, expert, a0.ctypes.data, a0.size,
                                           None if a1 is None else a1.ctypes.data, 0 if a1 is None else a1.size,
                                           empreinte_origine, empreinte_canonique, C.byref(en)))
        return en

    def terminer(self, entete: Entete) -> int:
        t = C.c_uint64()
        p, self._p = self._p, None
        _verifier(_l().trc_ecrivain_terminer(p, C.byref(entete), C.byref(t)))
        return int(t.value)

    def abandonner(self) -> None:
        if self._p:
            _l().trc_ecrivain_abandonner(self._p)
            self._p = None

    def __del__(self):
        try:
            self.abandonner()
        except Exception:
            pass
