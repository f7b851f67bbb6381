"""Host mirror of the native streaming scheduler (csrc/ordo.cpp): the expert path of the reference's
``Moteur`` (moteur/crates/trc-ordo/src/lib.rs:376-1280) over an opened .trc file, with the slot
cache in HBM. ``Ordonnanceur.jeton`` runs one token through every layer's MoE part.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from .cache import LRU, Compteurs
from .conteneur import Fichier, _verifier
from .noyaux import VueCarte, _flux, _statut, _vue, bibliotheque, _Vue  # noqa: F401


class ConfigOrdo(C.Structure):
    _fields_ = [("emplacements", C.c_uint32), ("tiedes", C.c_uint32), ("politique", C.c_int), ("verifier", C.c_int),
                ("lecteurs", C.c_uint32), ("prechargement", C.c_int), ("avec_biais_cache", C.c_int),
                ("biais_cache", C.c_float)]


class StatsOrdo(C.Structure):
    _fields_ = [("jetons", C.c_uint64), ("lectures", C.c_uint64), ("octets_lus", C.c_uint64),
                ("octets_copies", C.c_uint64), ("decodages", C.c_uint64), ("us_attente_routeur", C.c_double),
                ("us_lectures", C.c_double), ("us_emission", C.c_double), ("pf_emis", C.c_uint64),
                ("pf_utiles", C.c_uint64), ("pf_octets", C.c_uint64)]

    def dict(self) -> dict:
        return {n: getattr(self, n) for n, _t in self._fields_}


def _declarer(l):
    if getattr(l, "_trc_ordo", False):
        return l
    l.trc_ordo_creer.argtypes = [C.c_void_p, C.POINTER(ConfigOrdo), C.POINTER(C.c_void_p)]
    l.trc_ordo_jeton.argtypes = [C.c_void_p, _Vue, _Vue, C.c_void_p]
    l.trc_ordo_controle.argtypes = [C.c_void_p, C.POINTER(C.c_uint32), C.c_void_p]
    l.trc_ordo_compteurs.argtypes = [C.c_void_p]
    l.trc_ordo_compteurs.restype = Compteurs
    l.trc_ordo_stats.argtypes = [C.c_void_p]
    l.trc_ordo_stats.restype = StatsOrdo
    l.trc_ordo_trace.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64]
    l.trc_ordo_trace.restype = C.c_uint64
    l.trc_ordo_emplacement.argtypes = [C.c_void_p, C.c_uint16, C.c_uint16, C.POINTER(_Vue)]
    l.trc_ordo_temoin.argtypes = [C.c_void_p, C.c_uint16, C.c_uint16, C.c_void_p, C.POINTER(C.c_uint64)]
    l.trc_ordo_detruire.argtypes = [C.c_void_p]
    l._trc_ordo = True
    return l


def _l():
    return _declarer(bibliotheque())


class Ordonnanceur:
    """Moteur (trc-ordo/src/lib.rs:300-560), expert path. `emplacements` VRAM slots of decoded
    experts, `tiedes` pinned warm entries of coded parts (0: none), LRU or FIFO, `verifier`: each
    part read is checked against its directory fingerprint, `prechargement`: each layer predicts the
    next layer's experts and reads the predicted parts ahead (Config::prechargement), `biais_cache`:
    beta added to the router's score of the layer's experts already in VRAM for the choice of the k
    (Config::biais_cache; None: the plain router)."""

    def __init__(self, fichier: Fichier, emplacements: int, tiedes: int = 0, politique: int = LRU,
                 verifier: bool = False, lecteurs: int = 0, prechargement: bool = False,
                 biais_cache: float | None = None):
        self.fichier = fichier  # kept alive: the engine reads from it
        e = fichier.entete()
        self.L, self.E, self.k = e.couches, e.experts, e.k
        cfg = ConfigOrdo(emplacements, tiedes, politique, int(verifier), lecteurs, int(prechargement),
                         int(biais_cache is not None), 0.0 if biais_cache is None else float(biais_cache))
        p = C.c_void_p()
        _verifier(_l().trc_ordo_creer(fichier._p, C.byref(cfg), C.byref(p)))
        self._p = p

    def jeton(self, x, residu, f=None) -> None:
        _verifier(_l().trc_ordo_jeton(self._p, _vue(x), _vue(residu), _flux(f)))

    def controle(self, f=None) -> np.ndarray:
        m = (C.c_uint32 * 4)()
        _statut(_l().trc_ordo_controle(self._p, m, _flux(f)))
        return np.array(m[:], np.uint32)

    def compteurs(self) -> Compteurs:
        return _l().trc_ordo_compteurs(self._p)

    def stats(self) -> StatsOrdo:
        return _l().trc_ordo_stats(self._p)

    def trace(self) -> np.ndarray:
        """(jetons, couches, k) expert ids, in the order the router wrote them."""
        n = _l().trc_ordo_trace(self._p, None, 0)
        out = np.zeros(n, np.uint16)
        _l().trc_ordo_trace(self._p, out.ctypes.data, n)
        return out.reshape(-1, self.L, self.k)

    def emplacement(self, couche: int, expert: int) -> VueCarte:
        v = _Vue()
        _statut(_l().trc_ordo_emplacement(self._p, couche, expert, C.byref(v)))
        return VueCarte(v.adresse, v.octets)

    def temoin(self, couche: int, expert: int, f=None):
        """empreinte64 of the expert's decoded slot, or None if it is not in VRAM."""
        if _l().trc_ordo_emplacement(self._p, couche, expert, C.byref(_Vue())) != 0:
            return None
        e = C.c_uint64()
        _verifier(_l().trc_ordo_temoin(self._p, couche, expert, _flux(f), C.byref(e)))
        return int(e.value)

    def detruire(self) -> None:
        if self._p:
            _l().trc_ordo_detruire(self._p)
            self._p = C.c_void_p()

    def __del__(self):
        try:
            self.detruire()
        except Exception:
            pass
