"""Host mirror of the reference's model driver for one decode step (``trc_modele::Modele``,
moteur/crates/trc-modele/src/lib.rs:476-568) over this library's C-ABI: embedding row, then per
layer the attention half (``debut_couche``: RMSNorm, Q/K/V Q8_0 GEMVs, YaRN, f16 KV write, sink
attention, output projection, residual add, post-attention RMSNorm) and the MoE half
(``fin_couche``, here the fused compressed layer: router, top-k, rANS-decoded experts, SwiGLU and
the ordered combine into the residual), then the output head (RMSNorm, Q8_0 logits, argmax).
Same launch order and buffers as the reference; the cache slot of a position and the window of a
layer follow ``ParamsAttention::case`` / ``Hyper::anneau``.

Weights come from the caller as host arrays (``PoidsCouche``); ``poids_synthetiques`` draws a seeded
gpt-oss-shaped set (attention in Q8_0, experts coded by this library's encoder).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import codeur, fusion, noyaux
from .noyaux import DimsExpert, Noyaux, ParamsAttention, ParamsRope, VueCarte


@dataclass
class Hyper:
    """Hyper (trc-modele/src/lib.rs:60-79)."""
    couches: int
    d: int
    tetes: int
    tetes_kv: int
    experts: int
    actifs: int
    vocab: int
    eps: float
    rope: ParamsRope
    fenetre: int
    contexte: int
    dims: DimsExpert
    dt: int = 64
    n_delta: int = 4
    n_codes: int = 16
    # the synthetic model's gate and up matrices at other tile lengths than down (None: the same);
    # n_delta / n_codes, down's, are what the launches take
    n_delta_gu: int | None = None
    n_codes_gu: int | None = None

    def anneau(self, l: int) -> int:
        """lib.rs:140-143: the sliding window on even layers, the full cache on odd ones."""
        return self.fenetre if l % 2 == 0 else 0

    @property
    def dq(self) -> int:
        return self.tetes * self.dt

    @property
    def dkv(self) -> int:
        return self.tetes_kv * self.dt


@dataclass
class PoidsCouche:
    """One layer's weights on the host: attention in Q8_0 (rows of d/32 blocks of 34 bytes), norms,
    biases and sinks in f32, the router in bf16 (u16 bits, experts x d) with an optional f32 bias,
    and the experts as .trc v1.2 level-0 parts with their layer's frequency tables."""
    attn_norm: np.ndarray
    wq: np.ndarray
    bq: np.ndarray
    wk: np.ndarray
    bk: np.ndarray
    wv: np.ndarray
    bv: np.ndarray
    wo: np.ndarray
    bo: np.ndarray
    puits: np.ndarray
    post_norm: np.ndarray
    routeur: np.ndarray
    routeur_biais: np.ndarray | None
    parties: list = field(default_factory=list)
    freqs: list = field(default_factory=list)  # freqs[j][t]: 256 u16 or None


def _q8_0(rng, lignes: int, colonnes: int, echelle: float) -> np.ndarray:
    """A Q8_0 matrix of random int8 codes with f16 block scales around `echelle`."""
    nb = lignes * (colonnes // 32)
    d = (echelle * (1.0 + 0.1 * rng.standard_normal(nb))).astype(np.float16)
    q = rng.integers(-127, 128, size=(nb, 32)).astype(np.int8)
    return np.concatenate([d.view(np.uint8).reshape(-1, 2), q.view(np.uint8)], axis=1).ravel()


def _ech(c: int) -> float:
    return 1.0 / (73.0 * np.sqrt(c))  # |q| ~ 73 on average: rows of unit gain


def couche_synthetique(h: Hyper, graine: int, l: int, rng) -> PoidsCouche:
    """Layer `l` of a seeded model: attention drawn from `rng`, experts coded by the encoder."""
    d, dq, dkv = h.d, h.dq, h.dkv
    nd = h.n_delta if h.n_delta_gu is None else (h.n_delta_gu, h.n_delta_gu, h.n_delta)
    nc = h.n_codes if h.n_codes_gu is None else (h.n_codes_gu, h.n_codes_gu, h.n_codes)
    synth = codeur.CoucheSynthetique(graine, l, h.experts, h.dims, N_delta=nd, N_codes=nc)
    routeur = (rng.standard_normal((h.experts, d)) * (1.0 / np.sqrt(d))).astype(np.float32)
    p = PoidsCouche(
        attn_norm=(1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32),
        wq=_q8_0(rng, dq, d, _ech(d)), bq=(0.1 * rng.standard_normal(dq)).astype(np.float32),
        wk=_q8_0(rng, dkv, d, _ech(d)), bk=(0.1 * rng.standard_normal(dkv)).astype(np.float32),
        wv=_q8_0(rng, dkv, d, _ech(d)), bv=(0.1 * rng.standard_normal(dkv)).astype(np.float32),
        wo=_q8_0(rng, d, dq, _ech(dq)), bo=(0.1 * rng.standard_normal(d)).astype(np.float32),
        puits=rng.standard_normal(h.tetes).astype(np.float32),
        post_norm=(1.0 + 0.1 * rng.standard_normal(d)).astype(np.float32),
        routeur=(routeur.view(np.uint32) >> 16).astype(np.uint16),
        routeur_biais=(0.1 * rng.standard_normal(h.experts)).astype(np.float32),
        parties=[synth.partie(e).copy() for e in range(h.experts)],
        freqs=[[np.array(f) if f is not None else None for f in fj] for fj in synth.freqs()],
    )
    synth.liberer()
    return p


def tete_synthetique(h: Hyper, rng):
    """(embedding, output norm, output head) of a seeded model."""
    enchassement = _q8_0(rng, h.vocab, h.d, 0.02)
    norme_sortie = (1.0 + 0.1 * rng.standard_normal(h.d)).astype(np.float32)
    sortie = _q8_0(rng, h.vocab, h.d, _ech(h.d))
    return enchassement, norme_sortie, sortie


def poids_synthetiques(h: Hyper, graine: int):
    """Seeded weights of the shape `h`: (layers, embedding, output norm, output head)."""
    rng = np.random.default_rng(graine)
    couches = [couche_synthetique(h, graine, l, rng) for l in range(h.couches)]
    return (couches, *tete_synthetique(h, rng))


class _Tampons:
    """Device buffers (torch tensors as plumbing; the kernels see VueCarte)."""

    def __init__(self):
        import torch
        self._torch = torch
        self.garde = []

    def copie(self, a: np.ndarray):
        t = self._torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).to("cuda:0")
        self.garde.append(t)
        return t

    def zeros(self, octets: int):
        t = self._torch.zeros(octets, dtype=self._torch.uint8, device="cuda:0")
        self.garde.append(t)
        return t


def _v(t) -> VueCarte:
    return VueCarte.de(t)


class _Hyper(C.Structure):
    """trc_hyper (include/troncons_hip.h)."""
    _fields_ = [(n, C.c_uint32) for n in ("couches", "d", "tetes", "tetes_kv", "experts", "actifs", "vocab", "fenetre",
                                          "contexte", "n_delta", "n_codes")] + [
        ("eps", C.c_float), ("rope", ParamsRope), ("dims", DimsExpert)]


_CHAMPS_COUCHE = ("attn_norm", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "puits", "post_norm", "routeur",
                  "routeur_biais", "repertoire", "luts", "cache_k", "cache_v")


class _CoucheModele(C.Structure):
    """trc_couche_modele (include/troncons_hip.h)."""
    _fields_ = [(n, noyaux._Vue) for n in _CHAMPS_COUCHE]


def _declarer(l):
    if getattr(l, "_trc_modele", False):
        return l
    V = noyaux._Vue
    l.trc_modele_taille_travail.argtypes = [C.POINTER(_Hyper)]
    l.trc_modele_taille_travail.restype = C.c_uint64
    l.trc_modele_creer.argtypes = [C.POINTER(_Hyper), C.POINTER(_CoucheModele), V, V, V, V, C.POINTER(C.c_void_p)]
    l.trc_modele_detruire.argtypes = [C.c_void_p]
    l.trc_modele_vues.argtypes = [C.c_void_p] + [C.POINTER(V)] * 5
    l.trc_modele_enchasser.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p]
    l.trc_modele_couche.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p]
    l.trc_modele_sortie.argtypes = [C.c_void_p, C.c_void_p]
    l.trc_modele_pas.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p]
    l._trc_modele = True
    return l


class Modele:
    """Modele (lib.rs:366-602) for a model held resident: attention weights and KV caches in HBM,
    each layer's experts as resident coded parts mounted for the fused MoE layer."""

    def __init__(self, h: Hyper, couches: list, enchassement: np.ndarray, norme_sortie: np.ndarray,
                 sortie: np.ndarray, f=None):
        if h.dt != 64 or h.tetes % h.tetes_kv != 0 or h.d % 32 != 0:
            raise noyaux.ErreurUsage(f"forme d'attention {h.d} / {h.tetes} / {h.tetes_kv} / {h.dt}")
        if couches is not None and len(couches) != h.couches:
            raise noyaux.ErreurUsage(f"{len(couches)} couches pour {h.couches}")
        couches = couches or []
        self.h, self.f = h, f
        self.n, self.fz = Noyaux.charger(), fusion.Fusion()
        T = self.T = _Tampons()
        self.c = []
        for p in couches:
            self.ajouter_couche(p)
        self.emb, self.norme_sortie, self.w_sortie = T.copie(enchassement), T.copie(norme_sortie), T.copie(sortie)
        d, dq, dkv = h.d, h.dq, h.dkv
        self.x, self.hh, self.h2 = T.zeros(4 * d), T.zeros(4 * d), T.zeros(4 * d)
        self.q, self.k, self.v, self.a, self.o = T.zeros(4 * dq), T.zeros(4 * dkv), T.zeros(4 * dkv), T.zeros(4 * dq), T.zeros(4 * d)
        self.idx, self.pw = T.zeros(4 * 8), T.zeros(4 * 8)
        self.controle = T.zeros(16)
        self.travail = T.zeros(fusion.taille_travail_couche(h.dims, h.experts, h.actifs, h.n_codes) + 256)
        self.z, self.tok = T.zeros(4 * h.vocab), T.zeros(4)

    def ajouter_couche(self, p: PoidsCouche) -> None:
        """Uploads the next layer: attention weights, empty KV caches (the ring of a windowed layer,
        the context otherwise), the experts' parts mounted for the fused MoE layer, its LUTs."""
        h, T, f, l = self.h, self.T, self.f, len(self.c)
        c = {k: T.copie(getattr(p, k)) for k in ("attn_norm", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo",
                                                 "puits", "post_norm", "routeur")}
        c["routeur_biais"] = T.copie(p.routeur_biais) if p.routeur_biais is not None else None
        cases = h.anneau(l) or h.contexte
        c["ck"], c["cv"] = T.zeros(2 * cases * h.dkv), T.zeros(2 * cases * h.dkv)
        c["parties"] = [T.copie(np.asarray(pt, np.uint8)) for pt in p.parties]
        table = T.copie(np.array([t.data_ptr() for t in c["parties"]], np.uint64))
        c["rep"] = T.zeros(fusion.taille_repertoire(h.experts))
        ctl = T.zeros(16)
        self.fz.monter_couche(_v(table), h.experts, h.dims, _v(c["rep"]), _v(ctl), f)
        c["ctl_montage"] = ctl
        c["luts"] = T.copie(noyaux.luts_couche(p.freqs))
        self.c.append(c)

    @classmethod
    def synthetique(cls, h: Hyper, graine: int, progres=None, f=None) -> "Modele":
        """A seeded model of shape `h` built layer by layer (one layer's host copy at a time)."""
        rng = np.random.default_rng(graine)
        tete = tete_synthetique(h, rng)
        m = cls(h, None, *tete, f=f)
        for l in range(h.couches):
            m.ajouter_couche(couche_synthetique(h, graine, l, rng))
            if progres is not None:
                progres(l)
        return m

    def natif(self):
        """The native driver (csrc/modele.cpp) over this model's device buffers, created once the
        last layer is in: one C call per token."""
        if getattr(self, "_natif", None) is not None:
            return self._natif
        h = self.h
        if len(self.c) != h.couches:
            raise noyaux.ErreurUsage(f"{len(self.c)} couches montees sur {h.couches}")
        l = _declarer(noyaux.bibliotheque())
        hy = _Hyper(h.couches, h.d, h.tetes, h.tetes_kv, h.experts, h.actifs, h.vocab, h.fenetre, h.contexte,
                    h.n_delta, h.n_codes, h.eps, h.rope, h.dims)
        couches = (_CoucheModele * h.couches)()
        for i, c in enumerate(self.c):
            for n in _CHAMPS_COUCHE:
                t = {"repertoire": c["rep"], "cache_k": c["ck"], "cache_v": c["cv"]}.get(n, c.get(n))
                setattr(couches[i], n, noyaux._vue(t))
        octets = l.trc_modele_taille_travail(C.byref(hy))
        if octets == 0:
            raise noyaux.ErreurUsage("forme refusee par le pilote natif")
        self._travail_natif = self.T.zeros(octets + 256)
        tv = _v(self._travail_natif)
        dec = (-tv.adresse) % 256
        p = C.c_void_p()
        noyaux._statut(l.trc_modele_creer(C.byref(hy), couches, noyaux._vue(self.emb), noyaux._vue(self.norme_sortie),
                                          noyaux._vue(self.w_sortie), VueCarte(tv.adresse + dec, octets).c(),
                                          C.byref(p)))
        self._natif, self._l = p, l
        vues = [noyaux._Vue() for _ in range(5)]
        noyaux._statut(l.trc_modele_vues(p, *[C.byref(v) for v in vues]))
        self._vues_natif = [VueCarte(v.adresse, v.octets) for v in vues]
        return p

    def pas_natif(self, jeton: int, position: int) -> None:
        """trc_modele_pas: the same step issued by the native driver."""
        p = self.natif()
        noyaux._statut(self._l.trc_modele_pas(p, jeton, position, noyaux._flux(self.f)))

    def _lire_natif(self, i: int, dtype, n: int) -> np.ndarray:
        """Reads one of the native driver's buffers (a piece of the workspace tensor)."""
        import torch
        v = self._vues_natif[i]
        dec = v.adresse - self._travail_natif.data_ptr()
        octets = n * np.dtype(dtype).itemsize
        torch.cuda.synchronize()
        return self._travail_natif[dec:dec + octets].cpu().numpy().view(dtype).copy()

    def logits_natif(self) -> np.ndarray:
        return self._lire_natif(1, np.float32, self.h.vocab)

    def jeton_natif(self) -> int:
        return int(self._lire_natif(2, np.uint32, 1)[0])

    def controles_natif(self) -> np.ndarray:
        return self._lire_natif(4, np.uint32, 4)

    def __del__(self):
        try:
            if getattr(self, "_natif", None) is not None:
                self._l.trc_modele_detruire(self._natif)
                self._natif = None
        except Exception:
            pass

    def _travail(self) -> VueCarte:
        v = _v(self.travail)
        dec = (-v.adresse) % 256
        return VueCarte(v.adresse + dec, v.octets - dec)

    def enchasser(self, jeton: int) -> None:
        """lib.rs:481-487: x = row `jeton` of the Q8_0 embedding (exact)."""
        self.n.ligne_q8_0(_v(self.emb), jeton, self.h.d, _v(self.x), self.f)

    def attention_params(self, l: int, position: int) -> ParamsAttention:
        """ParamsAttention::gpt_oss (abi.rs:278-284) for this model's heads."""
        h, anneau = self.h, self.h.anneau(l)
        fin = position + 1
        debut = max(fin - anneau, 0) if anneau > 0 else 0
        return ParamsAttention(h.tetes, h.tetes_kv, 64, debut, fin, anneau, 1.0 / 8.0, 0)

    def debut_couche(self, l: int, position: int) -> None:
        """lib.rs:498-530, up to the post-attention norm; the router runs in the fused MoE half."""
        h, c, n, f = self.h, self.c[l], self.n, self.f
        if position >= h.contexte:
            raise noyaux.ErreurUsage(f"position {position} au-dela du contexte de {h.contexte} positions")
        d, dq, dkv = h.d, h.dq, h.dkv
        n.rmsnorm(_v(self.x), _v(c["attn_norm"]), _v(self.hh), d, 1, h.eps, f)
        n.gemv_q8_0(_v(c["wq"]), _v(self.hh), _v(c["bq"]), _v(self.q), dq, d, f)
        n.gemv_q8_0(_v(c["wk"]), _v(self.hh), _v(c["bk"]), _v(self.k), dkv, d, f)
        n.gemv_q8_0(_v(c["wv"]), _v(self.hh), _v(c["bv"]), _v(self.v), dkv, d, f)
        n.rope_yarn(_v(self.q), _v(self.k), h.tetes, h.tetes_kv, position, h.rope, f)
        n.ecrire_kv(_v(self.k), _v(self.v), _v(c["ck"]), _v(c["cv"]), dkv, ParamsAttention.case(position, h.anneau(l)), f)
        n.attention(_v(self.q), _v(c["ck"]), _v(c["cv"]), _v(c["puits"]), _v(self.a), self.attention_params(l, position), f)
        n.gemv_q8_0(_v(c["wo"]), _v(self.a), _v(c["bo"]), _v(self.o), d, dq, f)
        n.combiner(_v(self.x), _v(self.o), d, None, 1, d, f)
        n.rmsnorm(_v(self.x), _v(c["post_norm"]), _v(self.h2), d, 1, h.eps, f)

    def fin_couche(self, l: int) -> None:
        """lib.rs:530-555 with the router of lib.rs:523-528: the fused compressed MoE layer on h2,
        adding the ordered combine into x."""
        h, c = self.h, self.c[l]
        self.fz.couche_moe(_v(c["rep"]), h.experts, _v(c["luts"]), h.dims, _v(c["routeur"]),
                           _v(c["routeur_biais"]) if c["routeur_biais"] is not None else None, _v(self.h2), h.actifs,
                           _v(self.x), _v(self.idx), _v(self.pw), _v(self.controle), self._travail(), h.n_delta,
                           h.n_codes, self.f)

    def sortie(self) -> None:
        """lib.rs:557-568: RMSNorm, Q8_0 logits, greedy token (ties to the lower index)."""
        h, n, f = self.h, self.n, self.f
        n.rmsnorm(_v(self.x), _v(self.norme_sortie), _v(self.hh), h.d, 1, h.eps, f)
        n.gemv_q8_0(_v(self.w_sortie), _v(self.hh), None, _v(self.z), h.vocab, h.d, f)
        n.argmax(_v(self.z), h.vocab, _v(self.tok), f)

    def pas(self, jeton: int, position: int) -> None:
        """One decode step of token `jeton` at `position` through every layer (asynchronous)."""
        self.enchasser(jeton)
        for l in range(self.h.couches):
            self.debut_couche(l, position)
            self.fin_couche(l)
        self.sortie()

    def logits(self) -> np.ndarray:
        import torch
        torch.cuda.synchronize()
        return self.z.cpu().numpy().view(np.float32).copy()

    def jeton(self) -> int:
        import torch
        torch.cuda.synchronize()
        return int(self.tok.cpu().numpy().view(np.uint32)[0])

    def indices(self) -> np.ndarray:
        import torch
        torch.cuda.synchronize()
        return self.idx.cpu().numpy().view(np.uint32)[:self.h.actifs].copy()

    def controles(self) -> np.ndarray:
        import torch
        torch.cuda.synchronize()
        return np.concatenate([self.controle.cpu().numpy().view(np.uint32)] +
                              [c["ctl_montage"].cpu().numpy().view(np.uint32) for c in self.c])
