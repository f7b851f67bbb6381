"""Encoder front-end (host): synthetic gpt-oss-shape experts and .trc v1.2 level-0 parts, over the
C-ABI of libtroncons_hip.so (csrc/codeur.cpp). Plays the role of bins/trc-codeur for this build.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from .noyaux import DimsExpert, _statut, bibliotheque

_u8p = C.POINTER(C.c_uint8)
_f32p = C.POINTER(C.c_float)
_u16p = C.POINTER(C.c_uint16)


def _declarer(l):
    if getattr(l, "_trc_codeur", False):
        return l
    l.trc_synth_matrice.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _u8p, _f32p]
    l.trc_synth_normale_bf16.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_float, _f32p]
    l.trc_synth_expert.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.POINTER(DimsExpert), C.POINTER(_u8p),
                                   C.POINTER(_f32p)]
    l.trc_codeur_tables.argtypes = [C.POINTER(_u8p), C.c_uint32, C.c_uint32, C.c_uint32, C.c_int, _u16p]
    l.trc_codeur_partie.argtypes = [C.c_uint16, C.c_uint16, C.POINTER(DimsExpert), C.POINTER(_u8p), C.POINTER(_f32p),
                                    C.POINTER(_u16p), C.c_int, C.c_uint32, C.c_uint32, _u8p, C.c_uint64,
                                    C.POINTER(C.c_uint32)]
    l.trc_codeur_partie.restype = C.c_uint64
    l.trc_synth_couche.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.POINTER(DimsExpert), C.c_uint32, C.c_uint32,
                                   C.c_uint32]
    l.trc_synth_couche.restype = C.c_void_p
    l.trc_codeur_partie_n.argtypes = [C.c_uint16, C.c_uint16, C.POINTER(DimsExpert), C.POINTER(_u8p),
                                      C.POINTER(_f32p), C.POINTER(_u16p), C.c_int, C.POINTER(C.c_uint32),
                                      C.POINTER(C.c_uint32), _u8p, C.c_uint64, C.POINTER(C.c_uint32)]
    l.trc_codeur_partie_n.restype = C.c_uint64
    l.trc_synth_couche_n.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.POINTER(DimsExpert),
                                     C.POINTER(C.c_uint32), C.POINTER(C.c_uint32), C.c_uint32]
    l.trc_synth_couche_n.restype = C.c_void_p
    l.trc_synth_couche_taille.argtypes = [C.c_void_p, C.c_uint32]
    l.trc_synth_couche_taille.restype = C.c_uint64
    l.trc_synth_couche_utiles.argtypes = [C.c_void_p, C.c_uint32]
    l.trc_synth_couche_utiles.restype = C.c_uint32
    l.trc_synth_couche_partie.argtypes = [C.c_void_p, C.c_uint32]
    l.trc_synth_couche_partie.restype = C.c_void_p
    l.trc_synth_couche_freqs.argtypes = [C.c_void_p]
    l.trc_synth_couche_freqs.restype = C.c_void_p
    l.trc_synth_couche_liberer.argtypes = [C.c_void_p]
    l.trc_synth_couche_empreinte.argtypes = [C.c_void_p, C.c_uint32, C.c_int]
    l.trc_synth_couche_empreinte.restype = C.c_uint64
    l._trc_codeur = True
    return l


def _l():
    return _declarer(bibliotheque())


def _p(a, t):
    return a.ctypes.data_as(t)


def synth_matrice(graine: int, couche: int, expert: int, cle: int, R: int, C_: int):
    bl = np.zeros(17 * R * (C_ // 32), np.uint8)
    bi = np.zeros(R, np.float32)
    _l().trc_synth_matrice(graine, couche, expert, cle, R, C_, _p(bl, _u8p), _p(bi, _f32p))
    return bl, bi


def synth_normale_bf16(graine: int, cle1: int, cle2: int, n: int, sigma: float) -> np.ndarray:
    out = np.zeros(n, np.float32)
    _l().trc_synth_normale_bf16(graine, cle1, cle2, n, sigma, _p(out, _f32p))
    return out


def synth_expert(graine: int, couche: int, expert: int, dims: DimsExpert):
    bl = [np.zeros(17 * dims.lignes[j] * (dims.colonnes[j] // 32), np.uint8) for j in range(3)]
    bi = [np.zeros(dims.lignes[j], np.float32) for j in range(3)]
    pb = (_u8p * 3)(*[_p(a, _u8p) for a in bl])
    pi = (_f32p * 3)(*[_p(a, _f32p) for a in bi])
    _statut(_l().trc_synth_expert(graine, couche, expert, C.byref(dims), pb, pi))
    return bl, bi


def tables(blocs_experts, R: int, B: int, canonique: bool = True) -> np.ndarray:
    arrs = [np.ascontiguousarray(b, np.uint8) for b in blocs_experts]
    pb = (_u8p * len(arrs))(*[_p(a, _u8p) for a in arrs])
    out = np.zeros(1024, np.uint16)
    _statut(_l().trc_codeur_tables(pb, len(arrs), R, B, int(canonique), _p(out, _u16p)))
    return out.reshape(4, 256)


def par_matrice(N) -> "C.Array":
    """Tile lengths of the three matrices: one N for all, or (N_gate, N_up, N_down)."""
    t = [int(N)] * 3 if isinstance(N, (int, np.integer)) else [int(n) for n in N]
    assert len(t) == 3, N
    return (C.c_uint32 * 3)(*t)


def partie(blocs, biais, freqs, dims: DimsExpert, couche=0, expert=0, canonique=True, N_delta=256, N_codes=256):
    """A level-0 part; N_delta / N_codes: macro-steps per tile, one value or one per matrix."""
    bl = [np.ascontiguousarray(b, np.uint8) for b in blocs]
    bi = [np.ascontiguousarray(b, np.float32) for b in biais]
    fr = [np.ascontiguousarray(f, np.uint16).reshape(-1) for f in freqs]
    pb = (_u8p * 3)(*[_p(a, _u8p) for a in bl])
    pi = (_f32p * 3)(*[_p(a, _f32p) for a in bi])
    pf = (_u16p * 3)(*[_p(a, _u16p) for a in fr])
    u = C.c_uint32()
    args = (couche, expert, C.byref(dims), pb, pi, pf, int(canonique), par_matrice(N_delta), par_matrice(N_codes))
    n = _l().trc_codeur_partie_n(*args, _u8p(), 0, C.byref(u))
    if n == 0:
        _statut(1)
    out = np.zeros(n, np.uint8)
    _l().trc_codeur_partie_n(*args, _p(out, _u8p), n, C.byref(u))
    return out.tobytes(), u.value


def routage_zipf(graine: int, T: int, E: int, k: int, a: float = 1.1):
    """Config 5 routing: per position k distinct experts drawn from Zipf(a) over the E expert ranks
    without replacement (rank r = expert r), and the softmax weights of k seeded logits sorted in
    decreasing order (f64, rounded once to f32). Returns (indices u32[T, k], weights f32[T, k])."""
    rng = np.random.default_rng(graine)
    p = 1.0 / np.arange(1, E + 1, dtype=np.float64) ** a
    p /= p.sum()
    idx = np.zeros((T, k), np.uint32)
    w = np.zeros((T, k), np.float32)
    for i in range(T):
        idx[i] = rng.choice(E, size=k, replace=False, p=p)
        lg = np.sort(rng.standard_normal(k))[::-1]
        ex = np.exp(lg - lg[0])
        w[i] = (ex / ex.sum()).astype(np.float32)
    return idx, w


class CoucheSynthetique:
    """A synthetic layer: n experts' level-0 parts (v1.2) and the layer's tables."""

    def __init__(self, graine: int, couche: int, n_experts: int, dims: DimsExpert, N_delta: int = 256,
                 N_codes: int = 256, n_fils: int | None = None):
        if n_fils is None:
            n_fils = min(16, os.cpu_count() or 1)
        self.dims = dims
        self.n = n_experts
        self._h = _l().trc_synth_couche_n(graine, couche, n_experts, C.byref(dims), par_matrice(N_delta),
                                          par_matrice(N_codes), n_fils)
        if not self._h:
            _statut(1)

    def partie(self, e: int) -> np.ndarray:
        """The part of expert e (length a multiple of 4096), as a numpy view copied out."""
        n = _l().trc_synth_couche_taille(self._h, e)
        p = _l().trc_synth_couche_partie(self._h, e)
        return np.ctypeslib.as_array(C.cast(p, _u8p), shape=(n,)).copy()

    def utiles(self, e: int) -> int:
        return _l().trc_synth_couche_utiles(self._h, e)

    def taille(self, e: int) -> int:
        return _l().trc_synth_couche_taille(self._h, e)

    def empreinte(self, e: int, canonique: bool) -> int:
        """empreinte64 of expert e as generated, or with every nibble 8 of its codes set to 0."""
        return int(_l().trc_synth_couche_empreinte(self._h, e, int(canonique)))

    def freqs(self) -> np.ndarray:
        p = _l().trc_synth_couche_freqs(self._h)
        return np.ctypeslib.as_array(C.cast(p, _u16p), shape=(3, 4, 256)).copy()

    def liberer(self):
        if self._h:
            _l().trc_synth_couche_liberer(self._h)
            self._h = None

    def __del__(self):
        try:
            self.liberer()
        except Exception:
            pass
