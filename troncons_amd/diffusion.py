"""Host mirror of the streamed MoE layer on the fused path (csrc/diffusion.cpp): the experts' parts
in pinned host memory, per layer one mailbox wait, the k chosen parts copied on a side stream and
each decoded inside its fused MLP as soon as its copy lands (Moteur::pas with every part in RAM,
moteur/crates/trc-ordo/src/lib.rs:1054-1128, 1328-1370, without decoded slots).
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from .noyaux import DimsExpert, _flux, _statut, _vue, bibliotheque, _Vue  # noqa: F401


class CoucheHote(C.Structure):
    _fields_ = [("parties", C.c_void_p), ("decalages", C.POINTER(C.c_uint64)), ("tailles", C.POINTER(C.c_uint64)),
                ("luts", _Vue), ("routeur", _Vue)]


class StatsDiffusion(C.Structure):
    _fields_ = [("couches", C.c_uint64), ("octets_copies", C.c_uint64), ("us_attente_routeur", C.c_double)]

    def dict(self) -> dict:
        return {n: getattr(self, n) for n, _t in self._fields_}


def _declarer(l):
    if getattr(l, "_trc_diffusion", False):
        return l
    l.trc_diffusion_creer.argtypes = [C.POINTER(CoucheHote), C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(DimsExpert),
                                      C.c_uint32, C.c_uint32, C.POINTER(C.c_void_p)]
    l.trc_diffusion_couche.argtypes = [C.c_void_p, C.c_uint32, _Vue, _Vue, C.c_void_p, C.POINTER(C.c_uint32)]
    l.trc_diffusion_jeton.argtypes = [C.c_void_p, _Vue, _Vue, C.c_void_p]
    l.trc_diffusion_stats.argtypes = [C.c_void_p, C.POINTER(StatsDiffusion)]
    l.trc_diffusion_controle.argtypes = [C.c_void_p, C.POINTER(C.c_uint32)]
    l.trc_diffusion_detruire.argtypes = [C.c_void_p]
    l.trc_diffusion_detruire.restype = None
    l._trc_diffusion = True
    return l


def _l():
    return _declarer(bibliotheque())


class Diffusion:
    """The engine over layers given as (pinned host tensor of parts, offsets, lengths, LUTs view,
    f32 router view); every argument must outlive the engine (it keeps references)."""

    def __init__(self, couches, experts: int, k: int, dims: DimsExpert, n_delta: int, n_codes: int):
        self._l = _l()
        self._garde = []
        tab = (CoucheHote * len(couches))()
        for i, (parties, decalages, tailles, luts, routeur) in enumerate(couches):
            d = np.ascontiguousarray(decalages, np.uint64)
            t = np.ascontiguousarray(tailles, np.uint64)
            assert d.size == experts and t.size == experts
            self._garde += [parties, d, t, luts, routeur]
            tab[i] = CoucheHote(parties.data_ptr(), d.ctypes.data_as(C.POINTER(C.c_uint64)),
                                t.ctypes.data_as(C.POINTER(C.c_uint64)), _vue(luts), _vue(routeur))
        self.dims = dims
        self.k = k
        h = C.c_void_p()
        _statut(self._l.trc_diffusion_creer(tab, len(couches), experts, k, C.byref(dims), n_delta, n_codes,
                                            C.byref(h)))
        self.h = h

    def couche(self, l: int, x, residu, f=None) -> np.ndarray:
        """Layer l for x (residu += its combine); returns the k indices the router chose."""
        ch = (C.c_uint32 * self.k)()
        _statut(self._l.trc_diffusion_couche(self.h, l, _vue(x), _vue(residu), _flux(f), ch))
        return np.array(ch[:], np.uint32)

    def jeton(self, x, residu, f=None) -> None:
        _statut(self._l.trc_diffusion_jeton(self.h, _vue(x), _vue(residu), _flux(f)))

    def stats(self) -> dict:
        s = StatsDiffusion()
        _statut(self._l.trc_diffusion_stats(self.h, C.byref(s)))
        return s.dict()

    def controle(self) -> np.ndarray:
        m = (C.c_uint32 * 4)()
        _statut(self._l.trc_diffusion_controle(self.h, m))
        return np.array(m[:], np.uint32)

    def detruire(self) -> None:
        if self.h:
            self._l.trc_diffusion_detruire(self.h)
            self.h = C.c_void_p()
