"""Host mirror of the driver half of the launch layer (the reference's ``trc_cuda`` crate,
moteur/crates/trc-cuda/src/lib.rs:160-623): context, streams, events, device memory, pinned and
mapped host memory and the asynchronous copies, over the C-ABI of libtroncons_hip.so. Same names
as the reference's types and methods; no torch. A ``Flux`` has a ``cuda_stream`` attribute (its
hipStream_t), so it can be passed as ``f=`` to every launch method of ``Noyaux`` and ``Fusion``."""
from __future__ import annotations

import ctypes as C

import numpy as np

from .noyaux import VueCarte, _statut, _vue, _Vue, bibliotheque

ATTENTE_AUTO, ATTENTE_ACTIVE, ATTENTE_CEDE, ATTENTE_BLOQUANTE = 0, 1, 2, 3
(CAPACITE_MAJEURE, CAPACITE_MINEURE, MOTEURS_DE_COPIE, PROJECTION_HOTE, ADRESSAGE_UNIFIE, UNITES_DE_CALCUL,
 LDS_PAR_BLOC) = range(7)


def _declarer(l):
    if getattr(l, "_trc_pilote", False):
        return l
    P, V, u64p = C.c_void_p, _Vue, C.POINTER(C.c_uint64)
    l.trc_contexte_creer.argtypes = [C.c_uint32, C.c_uint32, C.POINTER(P)]
    l.trc_contexte_detruire.argtypes = [P]
    l.trc_contexte_detruire.restype = None
    l.trc_contexte_memoire.argtypes = [P, u64p, u64p]
    l.trc_contexte_nom.argtypes = [P]
    l.trc_contexte_nom.restype = C.c_char_p
    l.trc_contexte_version_pilote.argtypes = [P]
    l.trc_contexte_attente.argtypes = [P]
    l.trc_contexte_attente.restype = C.c_uint32
    l.trc_contexte_attribut.argtypes = [P, C.c_uint32, C.POINTER(C.c_int32)]
    l.trc_contexte_synchroniser.argtypes = [P]
    l.trc_flux_creer.argtypes = [P, C.c_int, C.POINTER(P)]
    l.trc_flux_detruire.argtypes = [P]
    l.trc_flux_attendre.argtypes = [P, P]
    l.trc_flux_synchroniser.argtypes = [P]
    l.trc_flux_fini.argtypes = [P, C.POINTER(C.c_int)]
    l.trc_flux_priorite.argtypes = [P, C.POINTER(C.c_int)]
    l.trc_evenement_creer.argtypes = [P, C.c_int, C.c_int, C.POINTER(P)]
    l.trc_evenement_detruire.argtypes = [P]
    l.trc_evenement_enregistrer.argtypes = [P, P]
    l.trc_evenement_fini.argtypes = [P, C.POINTER(C.c_int)]
    l.trc_evenement_attendre.argtypes = [P]
    l.trc_evenement_ms_depuis.argtypes = [P, P, C.POINTER(C.c_float)]
    l.trc_carte_allouer.argtypes = [P, C.c_uint64, C.POINTER(V)]
    l.trc_carte_liberer.argtypes = [P, V]
    l.trc_carte_remplir.argtypes = [V, C.c_uint8, P]
    l.trc_hote_allouer.argtypes = [P, C.c_uint64, C.c_int, C.POINTER(P), u64p, u64p]
    l.trc_hote_liberer.argtypes = [P]
    l.trc_hote_lire_volatil_u32.argtypes = [P, C.c_uint64]
    l.trc_hote_lire_volatil_u32.restype = C.c_uint32
    l.trc_copier_vers_carte.argtypes = [V, P, C.c_uint64, P]
    l.trc_copier_vers_hote.argtypes = [P, V, P]
    l.trc_copier_carte_carte.argtypes = [V, V, P]
    l._trc_pilote = True
    return l


def _l():
    return _declarer(bibliotheque())


class Contexte:
    """Contexte (lib.rs:160-247): device `ordinal`, host wait mode `attente` (ATTENTE_*)."""

    def __init__(self, ordinal: int = 0, attente: int = ATTENTE_AUTO):
        self._l = _l()
        h = C.c_void_p()
        _statut(self._l.trc_contexte_creer(ordinal, attente, C.byref(h)))
        self.h = h

    def memoire(self) -> tuple[int, int]:
        libre, totale = C.c_uint64(), C.c_uint64()
        _statut(self._l.trc_contexte_memoire(self.h, C.byref(libre), C.byref(totale)))
        return libre.value, totale.value

    def nom(self) -> str:
        return self._l.trc_contexte_nom(self.h).decode("utf-8", "replace")

    def version_pilote(self) -> int:
        return self._l.trc_contexte_version_pilote(self.h)

    def attente_effective(self) -> int:
        return self._l.trc_contexte_attente(self.h)

    def attribut(self, attribut: int) -> int:
        v = C.c_int32()
        _statut(self._l.trc_contexte_attribut(self.h, attribut, C.byref(v)))
        return v.value

    def synchroniser(self) -> None:
        _statut(self._l.trc_contexte_synchroniser(self.h))

    def detruire(self) -> None:
        if self.h:
            self._l.trc_contexte_detruire(self.h)
            self.h = None


class Flux:
    """Flux (lib.rs:278-340): a non-blocking stream at the default priority."""

    def __init__(self, c: Contexte, priorite_haute: bool = False):
        self._l = _l()
        h = C.c_void_p()
        _statut(self._l.trc_flux_creer(c.h, int(priorite_haute), C.byref(h)))
        self.h = h

    @property
    def cuda_stream(self) -> int:
        return self.h.value

    def attendre(self, e: "Evenement") -> None:
        _statut(self._l.trc_flux_attendre(self.h, e.h))

    def synchroniser(self) -> None:
        _statut(self._l.trc_flux_synchroniser(self.h))

    def fini(self) -> bool:
        f = C.c_int()
        _statut(self._l.trc_flux_fini(self.h, C.byref(f)))
        return bool(f.value)

    def priorite(self) -> int:
        p = C.c_int()
        _statut(self._l.trc_flux_priorite(self.h, C.byref(p)))
        return p.value

    def detruire(self) -> None:
        if self.h:
            _statut(self._l.trc_flux_detruire(self.h))
            self.h = None


class Evenement:
    """Evenement (lib.rs:348-423)."""

    def __init__(self, c: Contexte, horodate: bool = False, bloquant: bool = False):
        self._l = _l()
        h = C.c_void_p()
        _statut(self._l.trc_evenement_creer(c.h, int(horodate), int(bloquant), C.byref(h)))
        self.h = h

    def enregistrer(self, f: Flux) -> None:
        _statut(self._l.trc_evenement_enregistrer(self.h, f.h))

    def fini(self) -> bool:
        v = C.c_int()
        _statut(self._l.trc_evenement_fini(self.h, C.byref(v)))
        return bool(v.value)

    def attendre(self) -> None:
        _statut(self._l.trc_evenement_attendre(self.h))

    def ms_depuis(self, debut: "Evenement") -> float:
        ms = C.c_float()
        _statut(self._l.trc_evenement_ms_depuis(self.h, debut.h, C.byref(ms)))
        return ms.value

    def detruire(self) -> None:
        if self.h:
            _statut(self._l.trc_evenement_detruire(self.h))
            self.h = None


class MemoireCarte:
    """MemoireCarte (lib.rs:438-496): device memory owned by the caller."""

    def __init__(self, c: Contexte, octets: int):
        self._l = _l()
        self.c = c
        v = _Vue()
        _statut(self._l.trc_carte_allouer(c.h, octets, C.byref(v)))
        self.adresse, self.taille = v.adresse, v.octets

    def vue(self, decalage: int = 0, octets: int | None = None) -> VueCarte:
        n = self.taille - decalage if octets is None else octets
        assert 0 <= decalage and decalage + n <= self.taille, "vue hors de l'allocation"
        return VueCarte(self.adresse + decalage, n, self)

    def tout(self) -> VueCarte:
        return self.vue()

    def remplir(self, vue: VueCarte, octet: int, f: Flux) -> None:
        _statut(self._l.trc_carte_remplir(_vue(vue), octet, f.h))

    def liberer(self) -> None:
        if self.adresse:
            _statut(self._l.trc_carte_liberer(self.c.h, _Vue(self.adresse, self.taille)))
            self.adresse = 0


class HoteEpingle:
    """HoteEpingle (lib.rs:508-588): pinned host memory, mapped into the device if `projetee`."""

    def __init__(self, c: Contexte, octets: int, projetee: bool = False):
        self._l = _l()
        p, n, d = C.c_void_p(), C.c_uint64(), C.c_uint64()
        _statut(self._l.trc_hote_allouer(c.h, octets, int(projetee), C.byref(p), C.byref(n), C.byref(d)))
        self.p, self.taille, self.carte = p, n.value, (d.value or None)

    def tranche(self) -> np.ndarray:
        """The memory as a writable u8 array (no copy)."""
        return np.ctypeslib.as_array(C.cast(self.p, C.POINTER(C.c_uint8)), shape=(self.taille,))

    def adresse_carte(self) -> int | None:
        return self.carte

    def pointeur(self) -> int:
        return self.p.value

    def lire_volatil_u32(self, decalage: int) -> int:
        assert decalage % 4 == 0 and decalage + 4 <= self.taille, "lecture volatile hors limites"
        return self._l.trc_hote_lire_volatil_u32(self.p, decalage)

    def liberer(self) -> None:
        if self.p:
            _statut(self._l.trc_hote_liberer(self.p))
            self.p = None


def copier_vers_carte(dst: VueCarte, src: HoteEpingle, decalage: int, octets: int, f: Flux) -> None:
    """copier_vers_carte (lib.rs:591-603)."""
    if decalage + octets > src.taille:
        raise ValueError("copie vers la carte hors de la source")
    _statut(_l().trc_copier_vers_carte(_vue(dst), C.c_void_p(src.pointeur() + decalage), octets, f.h))


def copier_vers_hote(dst: HoteEpingle, decalage: int, src: VueCarte, f: Flux) -> None:
    """copier_vers_hote (lib.rs:606-614)."""
    if decalage + src.octets > dst.taille:
        raise ValueError("copie vers l'hote hors de la destination")
    _statut(_l().trc_copier_vers_hote(C.c_void_p(dst.pointeur() + decalage), _vue(src), f.h))


def copier_carte_carte(dst: VueCarte, src: VueCarte, f: Flux) -> None:
    """copier_carte_carte (lib.rs:617-623)."""
    _statut(_l().trc_copier_carte_carte(_vue(dst), _vue(src), f.h))
