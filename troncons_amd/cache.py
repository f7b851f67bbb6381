"""Host mirror of the expert slot cache and its simulator (the Rust crate ``trc_cache``,
moteur/crates/trc-cache/src), over the C-ABI of libtroncons_hip.so (csrc/cache.cpp).

Same names as the reference: ``Cache(...)`` (``Cache::nouveau``) / ``demander`` / ``pret`` / ``liberer`` /
``compteurs``, decisions ``Succes`` / ``DefautRam`` / ``DefautDisque``, ``Trace.depuis_texte``,
``rejouer``. A cache too small for the experts pinned at once raises ``ErreurUsage`` (the reference
panics); a malformed trace raises ``ErreurTrace`` with the reference's variant in ``classe``.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from .noyaux import ErreurUsage, _statut, bibliotheque

LRU, BELADY, FIFO = 0, 1, 2
LIBRE, EN_VOL, PRESENT = 0, 1, 2
SUCCES, DEFAUT_RAM, DEFAUT_DISQUE = 0, 1, 2
_CLASSES_TRACE = {32: "Ligne", 33: "HorsBornes", 34: "Vide"}


class ErreurTrace(ValueError):
    """ErreurTrace (trc-cache/src/trace.rs:140-152)"""

    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.classe = _CLASSES_TRACE.get(code, str(code))
        self.message = message


class _Decision(C.Structure):
    _fields_ = [("sorte", C.c_uint32), ("emplacement", C.c_uint32), ("tiede", C.c_int32), ("reserve", C.c_uint32)]


class Compteurs(C.Structure):
    """Compteurs (trc-cache/src/lib.rs:87-102) plus evictions_ram."""
    _fields_ = [("succes_vram", C.c_uint64), ("succes_ram", C.c_uint64), ("defauts_disque", C.c_uint64),
                ("octets_disque", C.c_uint64), ("octets_copies", C.c_uint64), ("evictions", C.c_uint64),
                ("evictions_ram", C.c_uint64)]

    def acces(self) -> int:
        return self.succes_vram + self.succes_ram + self.defauts_disque

    def tuple(self):
        return tuple(getattr(self, n) for n, _t in self._fields_)


@dataclass(frozen=True)
class Decision:
    """Decision (trc-cache/src/lib.rs:74-84): sorte SUCCES / DEFAUT_RAM / DEFAUT_DISQUE; tiede None
    when there is no warm entry."""
    sorte: int
    emplacement: int
    tiede: int | None


def _declarer(l):
    if getattr(l, "_trc_cache", False):
        return l
    l.trc_trace_depuis_texte.argtypes = [C.c_char_p, C.c_uint64, C.POINTER(C.c_void_p)]
    l.trc_trace_creer.argtypes = [C.c_uint16, C.c_uint16, C.c_uint16, C.c_uint32, C.c_void_p, C.POINTER(C.c_void_p)]
    l.trc_trace_dimensions.argtypes = [C.c_void_p, C.POINTER(C.c_uint32)]
    l.trc_trace_groupe.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32]
    l.trc_trace_groupe.restype = C.POINTER(C.c_uint16)
    l.trc_trace_liberer.argtypes = [C.c_void_p]
    l.trc_cache_creer.argtypes = [C.c_uint32, C.c_uint32, C.c_int, C.c_int, C.c_void_p, C.POINTER(C.c_void_p)]
    l.trc_cache_detruire.argtypes = [C.c_void_p]
    l.trc_cache_fixer_tailles.argtypes = [C.c_void_p, C.c_uint16, C.c_uint16, C.c_void_p]
    l.trc_cache_demander.argtypes = [C.c_void_p, C.c_uint16, C.c_void_p, C.c_uint32, C.c_uint64,
                                     C.POINTER(_Decision)]
    l.trc_cache_pret.argtypes = [C.c_void_p, C.c_uint32]
    l.trc_cache_liberer_couche.argtypes = [C.c_void_p, C.c_uint16]
    l.trc_cache_compteurs.argtypes = [C.c_void_p]
    l.trc_cache_compteurs.restype = Compteurs
    l.trc_cache_etat.argtypes = [C.c_void_p, C.c_uint32]
    l.trc_cache_occupant.argtypes = [C.c_void_p, C.c_uint32]
    l.trc_cache_occupant.restype = C.c_int64
    l.trc_cache_emplacement_de.argtypes = [C.c_void_p, C.c_uint16, C.c_uint16]
    l.trc_cache_emplacement_de.restype = C.c_int64
    l.trc_cache_tiede_de.argtypes = [C.c_void_p, C.c_uint16, C.c_uint16]
    l.trc_cache_tiede_de.restype = C.c_int64
    l.trc_cache_epingles.argtypes = [C.c_void_p, C.POINTER(C.c_uint32), C.c_uint32]
    l.trc_cache_epingles.restype = C.c_uint32
    l.trc_cache_ordre_vram.argtypes = [C.c_void_p, C.POINTER(C.c_uint32), C.c_uint32]
    l.trc_cache_ordre_vram.restype = C.c_uint32
    l.trc_cache_rejouer.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_int, C.c_int, C.POINTER(Compteurs)]
    l.trc_cache_rejouer_dans.argtypes = [C.c_void_p, C.c_void_p, C.POINTER(Compteurs)]
    l._trc_cache = True
    return l


def _l():
    return _declarer(bibliotheque())


def _id(v: int):
    return (v >> 16, v & 0xFFFF)


class Trace:
    """Trace (trc-cache/src/trace.rs:24-50): choix[(t * L + l) * k + i]."""

    def __init__(self, poignee: int, commentaires=()):
        self._p = C.c_void_p(poignee)
        d = (C.c_uint32 * 4)()
        _l().trc_trace_dimensions(self._p, d)
        self.experts, self.couches, self.k, self.jetons = (int(x) for x in d)
        self.commentaires = list(commentaires)

    @classmethod
    def depuis_texte(cls, texte: str) -> "Trace":
        b = texte.encode("utf-8")
        p = C.c_void_p()
        r = _l().trc_trace_depuis_texte(b, len(b), C.byref(p))
        if r in _CLASSES_TRACE:
            raise ErreurTrace(r, _l().trc_derniere_erreur().decode("utf-8", "replace"))
        _statut(r)
        com = [ligne.strip()[1:].strip() for ligne in texte.splitlines() if ligne.strip().startswith("#")]
        return cls(p.value, com)

    @classmethod
    def de(cls, experts: int, choix) -> "Trace":
        """choix: an array (jetons, couches, k) of expert ids."""
        a = np.ascontiguousarray(choix, np.uint16)
        assert a.ndim == 3
        p = C.c_void_p()
        _statut(_l().trc_trace_creer(experts, a.shape[1], a.shape[2], a.shape[0], a.ctypes.data, C.byref(p)))
        return cls(p.value)

    def groupe(self, jeton: int, couche: int) -> list:
        g = _l().trc_trace_groupe(self._p, jeton, couche)
        return [g[i] for i in range(self.k)]

    def acces(self) -> int:
        return self.jetons * self.couches * self.k

    def __del__(self):
        try:
            if self._p:
                _l().trc_trace_liberer(self._p)
                self._p = C.c_void_p()
        except Exception:
            pass


class Cache:
    """Cache (trc-cache/src/lib.rs:105-279), two stages: `emplacements` VRAM slots of decoded
    experts, `tiedes` warm-RAM entries of coded parts."""

    def __init__(self, emplacements: int, tiedes: int = 0, vram: int = LRU, ram: int = LRU, avenir: Trace | None = None):
        p = C.c_void_p()
        _statut(_l().trc_cache_creer(emplacements, tiedes, vram, ram, avenir._p if avenir else None, C.byref(p)))
        self._p = p
        self._avenir = avenir
        self.emplacements = emplacements

    def fixer_tailles(self, tailles) -> None:
        a = np.ascontiguousarray(tailles, np.uint64)
        _statut(_l().trc_cache_fixer_tailles(self._p, a.shape[0], a.shape[1], a.ctypes.data))

    def demander(self, couche: int, experts, t: int = 0) -> list:
        e = np.ascontiguousarray(experts, np.uint16)
        d = (_Decision * max(1, e.size))()
        _statut(_l().trc_cache_demander(self._p, couche, e.ctypes.data, e.size, t, d))
        return [Decision(d[i].sorte, d[i].emplacement, None if d[i].tiede < 0 else d[i].tiede) for i in range(e.size)]

    def pret(self, emplacement: int) -> None:
        _statut(_l().trc_cache_pret(self._p, emplacement))

    def liberer(self, couche: int) -> None:
        _l().trc_cache_liberer_couche(self._p, couche)

    def compteurs(self) -> Compteurs:
        return _l().trc_cache_compteurs(self._p)

    def etat(self, emplacement: int) -> int:
        return _l().trc_cache_etat(self._p, emplacement)

    def occupant(self, emplacement: int):
        v = _l().trc_cache_occupant(self._p, emplacement)
        return None if v < 0 else _id(v)

    def emplacement_de(self, couche: int, expert: int):
        v = _l().trc_cache_emplacement_de(self._p, couche, expert)
        return None if v < 0 else int(v)

    def tiede_de(self, couche: int, expert: int):
        v = _l().trc_cache_tiede_de(self._p, couche, expert)
        return None if v < 0 else int(v)

    def epingles(self) -> list:
        buf = (C.c_uint32 * 4096)()
        n = _l().trc_cache_epingles(self._p, buf, 4096)
        return [_id(buf[i]) for i in range(min(n, 4096))]

    def ordre_vram(self) -> list:
        buf = (C.c_uint32 * 65536)()
        n = _l().trc_cache_ordre_vram(self._p, buf, 65536)
        return [_id(buf[i]) for i in range(min(n, 65536))]

    def rejouer_dans(self, trace: Trace) -> Compteurs:
        c = Compteurs()
        _statut(_l().trc_cache_rejouer_dans(self._p, trace._p, C.byref(c)))
        return c

    def __del__(self):
        try:
            if self._p:
                _l().trc_cache_detruire(self._p)
                self._p = C.c_void_p()
        except Exception:
            pass


def rejouer(trace: Trace, emplacements: int, tiedes: int = 0, vram: int = LRU, ram: int = LRU) -> Compteurs:
    """rejouer (trc-cache/src/lib.rs:282-286): the simulator on a fresh cache."""
    c = Compteurs()
    _statut(_l().trc_cache_rejouer(trace._p, emplacements, tiedes, vram, ram, C.byref(c)))
    return c


__all__ = ["BELADY", "Cache", "Compteurs", "DEFAUT_DISQUE", "DEFAUT_RAM", "Decision", "EN_VOL", "ErreurTrace",
           "ErreurUsage", "FIFO", "LIBRE", "LRU", "PRESENT", "SUCCES", "Trace", "rejouer"]
