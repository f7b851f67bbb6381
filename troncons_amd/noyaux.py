"""Host mirror of the reference launch API (``trc_noyaux::Noyaux``, moteur/crates/trc-noyaux/src/lib.rs)
and of its ABI helpers (``trc_noyaux::abi``, moteur/crates/trc-noyaux/src/abi.rs), over the C-ABI of
libtroncons_hip.so.

Same method names, argument order and error behaviour as the reference: contract violations raise
``ErreurUsage`` before anything is launched, HIP failures raise ``ErreurHip``; data errors found by
kernels go to the caller's zeroed u32[4] control buffer. Device memory is borrowed through
``VueCarte`` (address, bytes); torch tensors are accepted as a convenience and converted to views.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

from . import _lib


class Erreur(RuntimeError):
    """trc_cuda::Erreur"""


class ErreurUsage(Erreur):
    """Erreur::Usage — contract violation found before any HIP call."""


class ErreurHip(Erreur):
    """Erreur::Cuda, on HIP — a runtime call failed; ``code`` is its hipError_t (the message holds
    the call, the runtime's error name and its text)."""

    def __init__(self, message: str, code: int = 0):
        super().__init__(message)
        self.code = code


class ErreurPilote(Erreur):
    """Erreur::Pilote — no usable HIP device."""


class _Vue(C.Structure):
    _fields_ = [("adresse", C.c_uint64), ("octets", C.c_uint64)]


class DimsExpert(C.Structure):
    """abi.rs:8-13 — 24 bytes, align 4."""
    _fields_ = [("lignes", C.c_uint32 * 3), ("colonnes", C.c_uint32 * 3)]

    @classmethod
    def de(cls, lignes, colonnes) -> "DimsExpert":
        d = cls()
        for j in range(3):
            d.lignes[j] = lignes[j]
            d.colonnes[j] = colonnes[j]
        return d

    @classmethod
    def gpt_oss(cls) -> "DimsExpert":
        return cls.de([2880] * 3, [2880] * 3)


class ParamsRope(C.Structure):
    """abi.rs:229-251 — YaRN parameters, 48 bytes."""
    _fields_ = [("base", C.c_double), ("facteur", C.c_double), ("ctx_origine", C.c_double),
                ("beta_rapide", C.c_double), ("beta_lent", C.c_double), ("dim_tete", C.c_uint32),
                ("variante", C.c_uint32)]

    @classmethod
    def gpt_oss(cls, **changes) -> "ParamsRope":
        """ParamsRope::GPT_OSS (abi.rs:249-250), fields overridable."""
        v = dict(base=150000.0, facteur=32.0, ctx_origine=4096.0, beta_rapide=32.0, beta_lent=1.0, dim_tete=64,
                 variante=0)
        v.update(changes)
        return cls(**v)


FENETRE_GPT_OSS = 128  # abi.rs:275


class ParamsAttention(C.Structure):
    """abi.rs:253-291 — one decode position's attention, 32 bytes."""
    _fields_ = [("tetes", C.c_uint32), ("tetes_kv", C.c_uint32), ("dim_tete", C.c_uint32), ("debut", C.c_uint32),
                ("fin", C.c_uint32), ("anneau", C.c_uint32), ("echelle", C.c_float), ("reserve", C.c_uint32)]

    @classmethod
    def gpt_oss(cls, position: int, fenetre: int) -> "ParamsAttention":
        """ParamsAttention::gpt_oss (abi.rs:278-284)."""
        fin = position + 1
        debut = max(fin - fenetre, 0) if fenetre > 0 else 0
        return cls(64, 8, 64, debut, fin, fenetre, 0.125, 0)

    @staticmethod
    def case(position: int, anneau: int) -> int:
        """abi.rs:287-289: the cache slot of a position."""
        return position % anneau if anneau > 0 else position


class DescGemv(C.Structure):
    """abi.rs:18-27 — 32 bytes."""
    _fields_ = [("matrice", C.c_uint64), ("x", C.c_uint64), ("y", C.c_uint64), ("lignes", C.c_uint32),
                ("colonnes", C.c_uint32)]


class DescDecodage(C.Structure):
    """abi.rs:33-42 — 32 bytes."""
    _fields_ = [("partie", C.c_uint64), ("emplacement", C.c_uint64), ("luts", C.c_uint64), ("controle", C.c_uint64)]

    def octets(self) -> bytes:
        return bytes(self)


class Disposition(C.Structure):
    """abi.rs:76-81"""
    _fields_ = [("base", C.c_uint64), ("echelles", C.c_uint64), ("biais", C.c_uint64), ("pas", C.c_uint64)]


@dataclass(frozen=True)
class VueCarte:
    """Non-owning view of device memory (trc-cuda/src/lib.rs:432-460). A view made from a torch
    tensor keeps that tensor alive as long as the view lives, so a temporary cannot be freed (and
    its memory handed to the next allocation) before the launch that borrows it is enqueued;
    stream order protects it afterwards."""
    adresse: int
    octets: int
    garde: object = field(default=None, compare=False, repr=False)

    @staticmethod
    def de(t, decalage: int = 0, octets: int | None = None) -> "VueCarte":
        """View of a torch tensor (or of a part of it, in bytes)."""
        total = t.numel() * t.element_size()
        n = total - decalage if octets is None else octets
        assert 0 <= decalage and decalage + n <= total
        return VueCarte(t.data_ptr() + decalage, n, t)

    def c(self) -> _Vue:
        return _Vue(self.adresse, self.octets)


AUCUNE = VueCarte(0, 0)


def _vue(v) -> _Vue:
    if v is None:
        return _Vue(0, 0)
    if isinstance(v, VueCarte):
        return v.c()
    return VueCarte.de(v).c()


def _declarer(l: C.CDLL) -> C.CDLL:
    if getattr(l, "_trc_declare", False):
        return l
    V = _Vue
    u32p = C.POINTER(C.c_uint32)
    l.trc_derniere_erreur.restype = C.c_char_p
    l.trc_dernier_code_hip.restype = C.c_int
    l.trc_disposition_matrice.argtypes = [C.c_uint32, C.c_uint32]
    l.trc_disposition_matrice.restype = Disposition
    l.trc_dims_verifier.argtypes = [C.POINTER(DimsExpert)]
    l.trc_disposition_j.argtypes = [C.POINTER(DimsExpert), C.c_uint32]
    l.trc_disposition_j.restype = Disposition
    l.trc_taille_emplacement.argtypes = [C.POINTER(DimsExpert)]
    l.trc_taille_emplacement.restype = C.c_uint64
    l.trc_grilles_decodeur.argtypes = [C.POINTER(DimsExpert), u32p, u32p]
    l.trc_grilles_depuis_partie.argtypes = [C.c_char_p, C.c_size_t, u32p, u32p]
    l.trc_grille_brut.argtypes = [C.POINTER(DimsExpert), u32p]
    l.trc_lut_geometrie1.argtypes = [C.POINTER(C.c_uint16), C.c_size_t, u32p]
    l.trc_luts_couche.argtypes = [C.POINTER(C.POINTER(C.c_uint16)), u32p]
    l.trc_decoder_expert.argtypes = [V, V, V, C.POINTER(DimsExpert), V, C.c_void_p]
    l.trc_decoder_expert_grilles.argtypes = [V, V, V, C.POINTER(DimsExpert), V, u32p, u32p, C.c_void_p]
    l.trc_decoder_lot.argtypes = [V, C.c_uint32, C.POINTER(DimsExpert), C.c_void_p]
    l.trc_copier_brut.argtypes = [V, V, C.POINTER(DimsExpert), V, C.c_void_p]
    l.trc_gemv.argtypes = [V, V, V, C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_gemv_lot.argtypes = [V, C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_gemv_f32.argtypes = [V, V, V, V, C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_routeur_topk.argtypes = [V, C.c_uint32, C.c_uint32, V, V, C.c_uint64, C.c_uint32, C.c_void_p]
    l.trc_routeur_topk_biais.argtypes = [V, V, C.c_uint32, C.c_uint32, V, V, C.c_uint64, C.c_uint32, C.c_void_p]
    l.trc_swiglu_oai.argtypes = [V, V, V, C.c_uint32, C.c_void_p]
    l.trc_combiner.argtypes = [V, V, C.c_uint32, V, C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_gemv_q8_0.argtypes = [V, V, V, V, C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_ligne_q8_0.argtypes = [V, C.c_uint32, C.c_uint32, V, C.c_void_p]
    l.trc_rmsnorm.argtypes = [V, V, V, C.c_uint32, C.c_uint32, C.c_float, C.c_void_p]
    l.trc_rope_yarn.argtypes = [V, V, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(ParamsRope), C.c_void_p]
    l.trc_ecrire_kv.argtypes = [V, V, V, V, C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_attention.argtypes = [V, V, V, V, V, C.POINTER(ParamsAttention), C.c_void_p]
    l.trc_ecrire_kv_f32.argtypes = [V, V, V, V, C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_attention_kvf32.argtypes = [V, V, V, V, V, C.POINTER(ParamsAttention), C.c_void_p]
    l.trc_argmax.argtypes = [V, C.c_uint32, V, C.c_void_p]
    l._trc_declare = True
    return l


def bibliotheque() -> C.CDLL:
    return _declarer(_lib.charger())


def _statut(r: int) -> None:
    if r == 0:
        return
    msg = bibliotheque().trc_derniere_erreur().decode("utf-8", "replace")
    if r == 1:
        raise ErreurUsage(msg)
    if r == 3:
        raise ErreurPilote(msg)
    raise ErreurHip(msg, bibliotheque().trc_dernier_code_hip())


def _flux(f) -> int:
    if f is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(f, int):
        return f
    return f.cuda_stream


# -------------------------------------------------------------------------------- abi helpers

def disposition_matrice(lignes: int, colonnes: int) -> Disposition:
    return bibliotheque().trc_disposition_matrice(lignes, colonnes)


def disposition(dims: DimsExpert, j: int) -> Disposition:
    return bibliotheque().trc_disposition_j(C.byref(dims), j)


def taille_emplacement(dims: DimsExpert) -> int:
    return bibliotheque().trc_taille_emplacement(C.byref(dims))


def verifier_dims(dims: DimsExpert) -> None:
    _statut(bibliotheque().trc_dims_verifier(C.byref(dims)))


def grilles_decodeur(dims: DimsExpert):
    g1 = (C.c_uint32 * 3)()
    g2 = (C.c_uint32 * 3)()
    bibliotheque().trc_grilles_decodeur(C.byref(dims), g1, g2)
    return list(g1), list(g2)


def grilles_depuis_partie(partie: bytes):
    g1 = (C.c_uint32 * 3)()
    g2 = (C.c_uint32 * 3)()
    _statut(bibliotheque().trc_grilles_depuis_partie(partie, len(partie), g1, g2))
    return list(g1), list(g2)


def grille_brut(dims: DimsExpert):
    g = (C.c_uint32 * 3)()
    bibliotheque().trc_grille_brut(C.byref(dims), g)
    return list(g)


def lut_geometrie1(freq):
    import numpy as np
    f = np.ascontiguousarray(freq, dtype=np.uint16)
    out = np.zeros(4096, dtype=np.uint32)
    _statut(bibliotheque().trc_lut_geometrie1(f.ctypes.data_as(C.POINTER(C.c_uint16)), f.size,
                                              out.ctypes.data_as(C.POINTER(C.c_uint32))))
    return out


def luts_couche(tables):
    """tables[j][t]: 256 frequencies or None -> u32[3*4*4096] (numpy)."""
    import numpy as np
    garde = []
    ptrs = (C.POINTER(C.c_uint16) * 12)()
    for j in range(3):
        for t in range(4):
            f = tables[j][t]
            if f is None:
                ptrs[j * 4 + t] = C.POINTER(C.c_uint16)()
            else:
                a = np.ascontiguousarray(f, dtype=np.uint16)
                if a.size != 256:
                    raise ErreurUsage(f"matrice {j}, table {t} : {a.size} fréquences")
                garde.append(a)
                ptrs[j * 4 + t] = a.ctypes.data_as(C.POINTER(C.c_uint16))
    out = np.zeros(3 * 4 * 4096, dtype=np.uint32)
    _statut(bibliotheque().trc_luts_couche(ptrs, out.ctypes.data_as(C.POINTER(C.c_uint32))))
    return out


# --------------------------------------------------------------------------------- launches

class Noyaux:
    """The kernels of the hot path, loaded once; every method launches asynchronously on ``f``
    (a torch stream, a raw hipStream_t as int, or None for torch's current stream)."""

    def __init__(self):
        self._l = bibliotheque()

    @classmethod
    def charger(cls) -> "Noyaux":
        return cls()

    def decoder_expert(self, partie, emplacement, luts, dims: DimsExpert, controle, f=None) -> None:
        """lib.rs:118"""
        _statut(self._l.trc_decoder_expert(_vue(partie), _vue(emplacement), _vue(luts), C.byref(dims),
                                           _vue(controle), _flux(f)))

    def decoder_expert_grilles(self, partie, emplacement, luts, dims: DimsExpert, controle, grilles, f=None) -> None:
        """lib.rs:142"""
        g1 = (C.c_uint32 * 3)(*grilles[0])
        g2 = (C.c_uint32 * 3)(*grilles[1])
        _statut(self._l.trc_decoder_expert_grilles(_vue(partie), _vue(emplacement), _vue(luts), C.byref(dims),
                                                   _vue(controle), g1, g2, _flux(f)))

    def decoder_lot(self, descs, n: int, dims: DimsExpert, f=None) -> None:
        """lib.rs:190"""
        _statut(self._l.trc_decoder_lot(_vue(descs), n, C.byref(dims), _flux(f)))

    def copier_brut(self, partie, emplacement, dims: DimsExpert, controle, f=None) -> None:
        """lib.rs:210"""
        _statut(self._l.trc_copier_brut(_vue(partie), _vue(emplacement), C.byref(dims), _vue(controle), _flux(f)))

    def gemv(self, matrice, x, y, lignes: int, colonnes: int, f=None) -> None:
        """lib.rs:239"""
        _statut(self._l.trc_gemv(_vue(matrice), _vue(x), _vue(y), lignes, colonnes, _flux(f)))

    def gemv_lot(self, descs, n: int, lignes_max: int, f=None) -> None:
        """lib.rs:274"""
        _statut(self._l.trc_gemv_lot(_vue(descs), n, lignes_max, _flux(f)))

    def gemv_f32(self, w, x, biais, y, lignes: int, colonnes: int, f=None) -> None:
        """lib.rs:307"""
        _statut(self._l.trc_gemv_f32(_vue(w), _vue(x), _vue(biais), _vue(y), lignes, colonnes, _flux(f)))

    def routeur_topk(self, logits, experts: int, k: int, indices, poids, boite: int = 0, sequence: int = 0,
                     f=None) -> None:
        """lib.rs:418"""
        _statut(self._l.trc_routeur_topk(_vue(logits), experts, k, _vue(indices), _vue(poids), boite, sequence,
                                         _flux(f)))

    def routeur_topk_biais(self, logits, biais, experts: int, k: int, indices, poids, boite: int = 0,
                           sequence: int = 0, f=None) -> None:
        """lib.rs:437"""
        _statut(self._l.trc_routeur_topk_biais(_vue(logits), _vue(biais), experts, k, _vue(indices), _vue(poids),
                                               boite, sequence, _flux(f)))

    def swiglu_oai(self, g, u, y, n: int, f=None) -> None:
        """lib.rs:451"""
        _statut(self._l.trc_swiglu_oai(_vue(g), _vue(u), _vue(y), n, _flux(f)))

    def combiner(self, residu, sorties, pas: int, poids, n: int, d: int, f=None) -> None:
        """lib.rs:463"""
        _statut(self._l.trc_combiner(_vue(residu), _vue(sorties), pas, _vue(poids), n, d, _flux(f)))

    # the rest of the layer step (passe.cuh)

    def gemv_q8_0(self, w, x, biais, y, lignes: int, colonnes: int, f=None) -> None:
        """lib.rs:291"""
        _statut(self._l.trc_gemv_q8_0(_vue(w), _vue(x), _vue(biais), _vue(y), lignes, colonnes, _flux(f)))

    def ligne_q8_0(self, w, ligne: int, colonnes: int, y, f=None) -> None:
        """lib.rs:478"""
        _statut(self._l.trc_ligne_q8_0(_vue(w), ligne, colonnes, _vue(y), _flux(f)))

    def rmsnorm(self, x, w, y, n: int, lignes: int, eps: float, f=None) -> None:
        """lib.rs:322"""
        _statut(self._l.trc_rmsnorm(_vue(x), _vue(w), _vue(y), n, lignes, eps, _flux(f)))

    def rope_yarn(self, q, k, tetes_q: int, tetes_k: int, position: int, p: ParamsRope, f=None) -> None:
        """lib.rs:334"""
        _statut(self._l.trc_rope_yarn(_vue(q), _vue(k), tetes_q, tetes_k, position, C.byref(p), _flux(f)))

    def ecrire_kv(self, k, v, cache_k, cache_v, dkv: int, case_kv: int, f=None) -> None:
        """lib.rs:348"""
        _statut(self._l.trc_ecrire_kv(_vue(k), _vue(v), _vue(cache_k), _vue(cache_v), dkv, case_kv, _flux(f)))

    def attention(self, q, cache_k, cache_v, puits, sortie, p: ParamsAttention, f=None) -> None:
        """lib.rs:362"""
        _statut(self._l.trc_attention(_vue(q), _vue(cache_k), _vue(cache_v), _vue(puits), _vue(sortie), C.byref(p),
                                      _flux(f)))

    def ecrire_kv_f32(self, k, v, cache_k, cache_v, dkv: int, case_kv: int, f=None) -> None:
        """lib.rs:383 (the trial f32 KV cache)"""
        _statut(self._l.trc_ecrire_kv_f32(_vue(k), _vue(v), _vue(cache_k), _vue(cache_v), dkv, case_kv, _flux(f)))

    def attention_kvf32(self, q, cache_k, cache_v, puits, sortie, p: ParamsAttention, f=None) -> None:
        """lib.rs:396 (the trial f32 KV cache)"""
        _statut(self._l.trc_attention_kvf32(_vue(q), _vue(cache_k), _vue(cache_v), _vue(puits), _vue(sortie),
                                            C.byref(p), _flux(f)))

    def argmax(self, v, n: int, sortie, f=None) -> None:
        """lib.rs:490"""
        _statut(self._l.trc_argmax(_vue(v), n, _vue(sortie), _flux(f)))
