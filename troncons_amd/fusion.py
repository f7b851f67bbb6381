"""Host mirror of the fused entry points (extensions of the launch API): one matrix, one expert
MLP, one MoE layer step, each decoding the rANS-coded part inside the GEMV kernels."""
from __future__ import annotations

import ctypes as C

from .noyaux import DimsExpert, _flux, _statut, _vue, _Vue, bibliotheque


def _declarer(l):
    if getattr(l, "_trc_fusion", False):
        return l
    V = _Vue
    l.trc_taille_travail_gemv_fusionnee.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32]
    l.trc_taille_travail_gemv_fusionnee.restype = C.c_uint64
    l.trc_gemv_fusionnee.argtypes = [V, C.c_uint32, V, C.c_uint32, C.c_uint32, V, V, V, V, C.c_uint32, C.c_uint32,
                                     C.c_void_p]
    l.trc_taille_travail_expert_fusionne.argtypes = [C.POINTER(DimsExpert), C.c_uint32]
    l.trc_taille_travail_expert_fusionne.restype = C.c_uint64
    l.trc_expert_fusionne.argtypes = [V, V, C.POINTER(DimsExpert), V, V, V, V, C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_taille_travail_couche_moe.argtypes = [C.POINTER(DimsExpert), C.c_uint32, C.c_uint32, C.c_uint32]
    l.trc_taille_travail_couche_moe.restype = C.c_uint64
    l.trc_couche_moe_fusionnee.argtypes = [V, C.c_uint32, V, C.POINTER(DimsExpert), V, V, V, C.c_uint32, V, V, V, V,
                                           V, C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_couche_moe_fusionnee_sans_alloc.argtypes = [V, C.c_uint32, V, C.POINTER(DimsExpert), V, V, V, C.c_uint32,
                                                      V, V, V, V, C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_octets_scratch.restype = C.c_uint64
    l.trc_taille_repertoire.argtypes = [C.c_uint32]
    l.trc_taille_repertoire.restype = C.c_uint64
    l.trc_monter_couche.argtypes = [V, C.c_uint32, C.POINTER(DimsExpert), V, V, C.c_void_p]
    l.trc_taille_travail_prefill.argtypes = [C.POINTER(DimsExpert), C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]
    l.trc_taille_travail_prefill.restype = C.c_uint64
    l.trc_prefill_moe.argtypes = [V, C.c_uint32, V, C.POINTER(DimsExpert), V, C.c_uint32, V, V, C.c_uint32, V, V, V,
                                  C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_chrono.argtypes = [C.c_int]
    l.trc_chrono_recolter.argtypes = [C.c_char_p, C.POINTER(C.c_double), C.POINTER(C.c_uint64), C.c_int, C.c_int]
    l._trc_fusion = True
    return l


def chrono(actif: bool) -> None:
    """Turns the per-kernel event chronogram of the fused entry points on or off."""
    _l().trc_chrono(int(actif))


def chrono_recolter(remettre_a_zero: bool = True) -> dict:
    """{kernel name: (total ms, launches)} of everything timed since the last reset."""
    n = 64
    noms = C.create_string_buffer(64 * n)
    ms = (C.c_double * n)()
    nb = (C.c_uint64 * n)()
    k = _l().trc_chrono_recolter(noms, ms, nb, n, int(remettre_a_zero))
    out = {}
    for i in range(k):
        nom = noms.raw[64 * i:64 * (i + 1)].split(b"\0", 1)[0].decode()
        out[nom] = (ms[i], nb[i])
    return out


def _l():
    return _declarer(bibliotheque())


def taille_travail_gemv(lignes: int, colonnes: int, n_codes: int) -> int:
    return _l().trc_taille_travail_gemv_fusionnee(lignes, colonnes, n_codes)


def taille_travail_expert(dims: DimsExpert, n_codes: int) -> int:
    return _l().trc_taille_travail_expert_fusionne(C.byref(dims), n_codes)


def taille_travail_couche(dims: DimsExpert, experts: int, k: int, n_codes: int) -> int:
    return _l().trc_taille_travail_couche_moe(C.byref(dims), experts, k, n_codes)


def taille_travail_prefill(dims: DimsExpert, experts: int, positions: int, k: int, n_codes: int) -> int:
    return _l().trc_taille_travail_prefill(C.byref(dims), experts, positions, k, n_codes)


def octets_scratch() -> int:
    """Bytes of the static device scratch of couche_moe_sans_alloc."""
    return _l().trc_octets_scratch()


def taille_repertoire(experts: int) -> int:
    """Bytes of a mounted layer's directory (trc_monter_couche)."""
    return _l().trc_taille_repertoire(experts)


class Fusion:
    """Fused hot path; every call is asynchronous on ``f`` (torch stream, hipStream_t int, or None
    for torch's current stream)."""

    def __init__(self):
        self._l = _l()

    def gemv_fusionnee(self, partie, j: int, luts, lignes: int, colonnes: int, x, y, controle, travail,
                       n_delta: int, n_codes: int, f=None) -> None:
        _statut(self._l.trc_gemv_fusionnee(_vue(partie), j, _vue(luts), lignes, colonnes, _vue(x), _vue(y),
                                           _vue(controle), _vue(travail), n_delta, n_codes, _flux(f)))

    def expert_fusionne(self, partie, luts, dims: DimsExpert, x, sortie, controle, travail, n_delta: int,
                        n_codes: int, f=None) -> None:
        _statut(self._l.trc_expert_fusionne(_vue(partie), _vue(luts), C.byref(dims), _vue(x), _vue(sortie),
                                            _vue(controle), _vue(travail), n_delta, n_codes, _flux(f)))

    def monter_couche(self, parties, experts: int, dims: DimsExpert, repertoire, controle, f=None) -> None:
        """Parses the experts' parts (u64[experts] device addresses) once into `repertoire`."""
        _statut(self._l.trc_monter_couche(_vue(parties), experts, C.byref(dims), _vue(repertoire), _vue(controle),
                                          _flux(f)))

    def couche_moe(self, repertoire, experts: int, luts, dims: DimsExpert, routeur, routeur_biais, x, k: int, residu,
                   indices, poids, controle, travail, n_delta: int, n_codes: int, f=None) -> None:
        _statut(self._l.trc_couche_moe_fusionnee(_vue(repertoire), experts, _vue(luts), C.byref(dims), _vue(routeur),
                                                 _vue(routeur_biais), _vue(x), k, _vue(residu), _vue(indices),
                                                 _vue(poids), _vue(controle), _vue(travail), n_delta, n_codes,
                                                 _flux(f)))

    def couche_moe_sans_alloc(self, repertoire, experts: int, luts, dims: DimsExpert, routeur, routeur_biais, x,
                              k: int, residu, indices, poids, controle, n_delta: int, n_codes: int, f=None) -> None:
        """couche_moe with the library's static device scratch as workspace (no allocation; calls
        that overlap on one device race)."""
        _statut(self._l.trc_couche_moe_fusionnee_sans_alloc(
            _vue(repertoire), experts, _vue(luts), C.byref(dims), _vue(routeur), _vue(routeur_biais), _vue(x), k,
            _vue(residu), _vue(indices), _vue(poids), _vue(controle), n_delta, n_codes, _flux(f)))

    def prefill_moe(self, repertoire, experts: int, luts, dims: DimsExpert, x, positions: int, indices, poids, k: int,
                    residus, controle, travail, n_delta: int, n_codes: int, f=None) -> None:
        """Batched prefill of one resident layer: residus[i] += the weighted outputs of position i's
        k experts (indices / poids: [positions][k])."""
        _statut(self._l.trc_prefill_moe(_vue(repertoire), experts, _vue(luts), C.byref(dims), _vue(x), positions,
                                        _vue(indices), _vue(poids), k, _vue(residus), _vue(controle), _vue(travail),
                                        n_delta, n_codes, _flux(f)))
