"""ctypes binding of the CPU oracle (oracle/liboracle.so) — test infrastructure.

Only tests, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg use this module, as the
checker or as the timed CPU baseline; the product never does.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib
import subprocess

import numpy as np

RACINE = pathlib.Path(__file__).resolve().parents[1]
ORACLE = RACINE / "oracle"
LIB_PATH = ORACLE / "liboracle.so"

M = 4096
L = 1 << 16


def construire() -> None:
    """make -C oracle (idempotent)."""
    subprocess.run(["make", "-s", "-C", str(ORACLE)], check=True)


def _charger() -> C.CDLL:
    if not LIB_PATH.exists():
        construire()
    return C.CDLL(str(LIB_PATH))


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        _lib = _charger()
        _declarer(_lib)
    return _lib


u8p = C.POINTER(C.c_uint8)
u16p = C.POINTER(C.c_uint16)
u32p = C.POINTER(C.c_uint32)
u64p = C.POINTER(C.c_uint64)
f32p = C.POINTER(C.c_float)
f64p = C.POINTER(C.c_double)


class Flux(C.Structure):
    _fields_ = [("P", C.c_uint32), ("N", C.c_uint32), ("geometrie", C.c_uint32), ("T", C.c_uint32),
                ("W", C.c_uint32), ("debuts", u8p), ("etats", u8p), ("mots", u8p)]


class Bilan(C.Structure):
    _fields_ = [("voies_hors_l", C.c_uint64), ("tuiles_mots_faux", C.c_uint64), ("premiere_tuile", C.c_int64)]


class DescFlux(C.Structure):
    _fields_ = [("sorte", C.c_uint8), ("matrice", C.c_uint8), ("contexte", C.c_uint8),
                ("decalage", C.c_uint32), ("longueur", C.c_uint32), ("produits", C.c_uint32)]


class Partie(C.Structure):
    _fields_ = [("couche", C.c_uint16), ("expert", C.c_uint16), ("niveau", C.c_uint8), ("n_matrices", C.c_uint8),
                ("n_flux", C.c_uint32), ("utiles", C.c_uint32), ("flux", DescFlux * 64)]


class ParamsRope(C.Structure):
    """ParamsRope (trc-noyaux/src/abi.rs:229-251): 48 bytes."""
    _fields_ = [("base", C.c_double), ("facteur", C.c_double), ("ctx_origine", C.c_double),
                ("beta_rapide", C.c_double), ("beta_lent", C.c_double), ("dim_tete", C.c_uint32),
                ("variante", C.c_uint32)]


def rope_gpt_oss(**k) -> ParamsRope:
    """ParamsRope::GPT_OSS (abi.rs:249-250), fields overridable."""
    v = dict(base=150000.0, facteur=32.0, ctx_origine=4096.0, beta_rapide=32.0, beta_lent=1.0, dim_tete=64, variante=0)
    v.update(k)
    return ParamsRope(**v)


class ParamsAttention(C.Structure):
    """ParamsAttention (abi.rs:253-291): 32 bytes."""
    _fields_ = [("tetes", C.c_uint32), ("tetes_kv", C.c_uint32), ("dim_tete", C.c_uint32), ("debut", C.c_uint32),
                ("fin", C.c_uint32), ("anneau", C.c_uint32), ("echelle", C.c_float), ("reserve", C.c_uint32)]


def attention_gpt_oss(position: int, fenetre: int, tetes: int = 64, tetes_kv: int = 8) -> ParamsAttention:
    """ParamsAttention::gpt_oss (abi.rs:278-284)."""
    fin = position + 1
    debut = max(fin - fenetre, 0) if fenetre > 0 else 0
    return ParamsAttention(tetes, tetes_kv, 64, debut, fin, fenetre, 0.125, 0)


class Disposition(C.Structure):
    _fields_ = [("base", C.c_uint64), ("echelles", C.c_uint64), ("biais", C.c_uint64), ("pas", C.c_uint64)]


def _declarer(l: C.CDLL) -> None:
    l.orc_table_depuis_comptes.argtypes = [u64p, C.c_int, u16p]
    l.orc_lut.argtypes = [u16p, C.c_int, u32p, u32p]
    l.orc_lut.restype = C.c_int
    l.orc_luts_couche.argtypes = [C.POINTER(u16p), u32p]
    l.orc_flux_lire.argtypes = [u8p, C.c_size_t, C.POINTER(Flux)]
    l.orc_coder.argtypes = [u8p, C.c_size_t, C.c_int, u8p, C.c_size_t, u16p, C.c_int, C.c_uint32, u8p, C.c_size_t]
    l.orc_coder.restype = C.c_size_t
    l.orc_decoder.argtypes = [C.POINTER(Flux), u8p, C.c_size_t, u32p, C.c_int, u8p, C.POINTER(Bilan)]
    l.orc_classe_echelle.argtypes = [C.c_uint8]
    l.orc_classe_echelle.restype = C.c_uint8
    l.orc_canoniser_octet.argtypes = [C.c_uint8]
    l.orc_canoniser_octet.restype = C.c_uint8
    l.orc_preparer_matrice.argtypes = [u8p, C.c_uint32, C.c_uint32, C.c_int, u8p, u8p, u8p]
    l.orc_comptes_ajouter.argtypes = [u8p, C.c_size_t, u8p, C.c_size_t, u64p, u64p]
    l.orc_assembler_partie.argtypes = [C.c_uint16, C.c_uint16, C.c_uint8, C.c_uint8, C.c_int, u8p, u8p, u8p, u32p,
                                       C.POINTER(u8p), u32p, u8p, C.c_size_t, u32p]
    l.orc_assembler_partie.restype = C.c_size_t
    l.orc_lire_partie.argtypes = [u8p, C.c_size_t, C.POINTER(Partie)]
    l.orc_coder_expert.argtypes = [C.c_uint16, C.c_uint16, C.c_int, u32p, u32p, C.POINTER(u8p), C.POINTER(u8p),
                                   C.POINTER(u16p), C.c_int, C.c_uint32, C.c_uint32, u8p, C.c_size_t, u32p]
    l.orc_coder_expert.restype = C.c_size_t
    l.orc_tables_matrice.argtypes = [C.POINTER(u8p), C.c_int, C.c_uint32, C.c_uint32, C.c_int, u16p]
    l.orc_decoder_matrice.argtypes = [u8p, C.c_size_t, C.c_uint8, C.c_uint32, C.c_uint32, u32p, u8p, u8p, u8p,
                                      C.POINTER(Bilan), C.POINTER(Bilan)]
    l.orc_disposition_matrice.argtypes = [C.c_uint32, C.c_uint32]
    l.orc_disposition_matrice.restype = Disposition
    l.orc_taille_emplacement.argtypes = [u32p, u32p]
    l.orc_taille_emplacement.restype = C.c_uint64
    l.orc_disposition_j.argtypes = [u32p, u32p, C.c_int]
    l.orc_disposition_j.restype = Disposition
    l.orc_decoder_expert.argtypes = [u8p, C.c_size_t, u32p, u32p, u32p, u8p, u32p]
    l.orc_echelle_e8m0.argtypes = [C.c_uint32]
    l.orc_echelle_e8m0.restype = C.c_float
    l.orc_valeur_e2m1x2.argtypes = [C.c_uint32]
    l.orc_valeur_e2m1x2.restype = C.c_float
    l.orc_gemv_mxfp4.argtypes = [u8p, f32p, f32p, C.c_uint32, C.c_uint32]
    l.orc_gemv_mxfp4_f64.argtypes = [u8p, f32p, f64p, C.c_uint32, C.c_uint32]
    l.orc_gemv_f32.argtypes = [f32p, f32p, f32p, f32p, C.c_uint32, C.c_uint32]
    l.orc_swiglu_oai.argtypes = [f32p, f32p, f32p, C.c_uint32]
    l.orc_combiner.argtypes = [f32p, f32p, C.c_uint32, f32p, C.c_uint32, C.c_uint32]
    l.orc_routeur_topk.argtypes = [f32p, C.c_uint32, C.c_uint32, u32p, f32p]
    l.orc_routeur_topk_biais.argtypes = [f32p, f32p, C.c_uint32, C.c_uint32, u32p, f32p]
    l.orc_f32_depuis_f16.argtypes = [C.c_uint16]
    l.orc_f32_depuis_f16.restype = C.c_float
    l.orc_f16_depuis_f32.argtypes = [C.c_float]
    l.orc_f16_depuis_f32.restype = C.c_uint16
    l.orc_gemv_q8_0.argtypes = [u8p, f32p, f32p, f32p, C.c_uint32, C.c_uint32]
    l.orc_ligne_q8_0.argtypes = [u8p, C.c_uint32, C.c_uint32, f32p]
    l.orc_rmsnorm.argtypes = [f32p, f32p, f32p, C.c_uint32, C.c_uint32, C.c_float]
    l.orc_inv_freq_yarn.argtypes = [C.POINTER(ParamsRope), C.c_uint32, f64p, f64p, f64p]
    l.orc_inv_freq_yarn.restype = C.c_double
    l.orc_rope_yarn.argtypes = [f32p, f32p, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(ParamsRope)]
    l.orc_ecrire_kv.argtypes = [f32p, f32p, u16p, u16p, C.c_uint32, C.c_uint32]
    l.orc_attention.argtypes = [f32p, u16p, u16p, f32p, f32p, C.POINTER(ParamsAttention)]
    l.orc_argmax.argtypes = [f32p, C.c_uint32]
    l.orc_argmax.restype = C.c_uint32
    l.orc_splitmix64.argtypes = [u64p]
    l.orc_splitmix64.restype = C.c_uint64
    l.orc_xorshift64s.argtypes = [u64p]
    l.orc_xorshift64s.restype = C.c_uint64
    l.orc_bf16_depuis_f32.argtypes = [C.c_float]
    l.orc_bf16_depuis_f32.restype = C.c_uint16
    l.orc_f32_depuis_bf16.argtypes = [C.c_uint16]
    l.orc_f32_depuis_bf16.restype = C.c_float
    l.orc_synth_matrice.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, u8p, f32p]
    l.orc_synth_normale_bf16.argtypes = [C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32, C.c_float, f32p]
    l.orc_empreinte64.argtypes = [u8p, C.c_size_t]
    l.orc_empreinte64.restype = C.c_uint64


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(t)


# ------------------------------------------------------------------------------ python-level API

def table_depuis_comptes(comptes, geometrie: int = 1) -> np.ndarray:
    n = 256 if geometrie == 1 else 16
    c = np.ascontiguousarray(comptes, dtype=np.uint64)
    assert c.size == n
    f = np.zeros(n, dtype=np.uint16)
    lib().orc_table_depuis_comptes(_p(c, u64p), geometrie, _p(f, u16p))
    return f


def lut(freq, geometrie: int = 1):
    """Returns (cumul, lut) or None when the frequencies are refused."""
    f = np.ascontiguousarray(freq, dtype=np.uint16)
    cum = np.zeros(f.size, dtype=np.uint32)
    l = np.zeros(M, dtype=np.uint32)
    if lib().orc_lut(_p(f, u16p), geometrie, _p(cum, u32p), _p(l, u32p)) != 0:
        return None
    return cum, l


def luts_couche(freqs) -> np.ndarray:
    """freqs: 3x4 nested list of 256-u16 arrays or None -> u32[3*4*4096]."""
    arrs = []
    ptrs = (u16p * 12)()
    for j in range(3):
        for t in range(4):
            f = freqs[j][t]
            if f is None:
                ptrs[j * 4 + t] = u16p()
            else:
                a = np.ascontiguousarray(f, dtype=np.uint16)
                arrs.append(a)
                ptrs[j * 4 + t] = _p(a, u16p)
    out = np.zeros(3 * 4 * M, dtype=np.uint32)
    if lib().orc_luts_couche(ptrs, _p(out, u32p)) != 0:
        raise ValueError("table refused")
    return out


def coder(source: np.ndarray, freqs: np.ndarray, geometrie: int = 1, kappa=None, N: int = 256) -> bytes:
    src = np.ascontiguousarray(source, dtype=np.uint8)
    fr = np.ascontiguousarray(freqs, dtype=np.uint16)
    n_sym = 256 if geometrie == 1 else 16
    ntab = fr.size // n_sym
    kp = np.ascontiguousarray(kappa, dtype=np.uint8) if kappa is not None else None
    args = (_p(src, u8p), src.size, geometrie, _p(kp, u8p) if kp is not None else u8p(),
            kp.size if kp is not None else 0, _p(fr, u16p), ntab, N)
    n = lib().orc_coder(*args, u8p(), 0)
    if n == 0:
        raise ValueError("encoding refused")
    out = np.zeros(n, dtype=np.uint8)
    lib().orc_coder(*args, _p(out, u8p), n)
    return out.tobytes()


def flux_lire(b: bytes):
    buf = np.frombuffer(b, dtype=np.uint8).copy()
    f = Flux()
    if lib().orc_flux_lire(_p(buf, u8p), buf.size, C.byref(f)) != 0:
        return None
    f._garde = buf  # keep the buffer alive
    return f


def decoder(flux_octets: bytes, luts: np.ndarray, kappa=None):
    """Returns (decoded bytes, Bilan) or raises on a refused stream."""
    f = flux_lire(flux_octets)
    if f is None:
        raise ValueError("stream refused")
    lt = np.ascontiguousarray(luts, dtype=np.uint32)
    kp = np.ascontiguousarray(kappa, dtype=np.uint8) if kappa is not None else None
    out = np.zeros(f.P, dtype=np.uint8)
    b = Bilan()
    r = lib().orc_decoder(C.byref(f), _p(kp, u8p) if kp is not None else u8p(), kp.size if kp is not None else 0,
                          _p(lt, u32p), lt.size // M, _p(out, u8p), C.byref(b))
    if r != 0:
        raise ValueError("context without table")
    return out, b


def preparer_matrice(blocs17: np.ndarray, R: int, B: int, canonique: bool = False):
    nb = R * B
    med = np.zeros(R, dtype=np.uint8)
    delta = np.zeros(-(-nb // 128) * 128, dtype=np.uint8)
    qs = np.zeros(-(-(16 * nb) // 128) * 128, dtype=np.uint8)
    bl = np.ascontiguousarray(blocs17, dtype=np.uint8)
    lib().orc_preparer_matrice(_p(bl, u8p), R, B, int(canonique), _p(med, u8p), _p(delta, u8p), _p(qs, u8p))
    return med, delta, qs


def tables_matrice(blocs_experts, R: int, B: int, canonique: bool = True) -> np.ndarray:
    arrs = [np.ascontiguousarray(b, dtype=np.uint8) for b in blocs_experts]
    ptrs = (u8p * len(arrs))(*[_p(a, u8p) for a in arrs])
    out = np.zeros(4 * 256, dtype=np.uint16)
    lib().orc_tables_matrice(ptrs, len(arrs), R, B, int(canonique), _p(out, u16p))
    return out.reshape(4, 256)


def assembler_partie(couche, expert, niveau, n_matrices, flux):
    """flux: list of (sorte, matrice, contexte, produits, bytes). Returns (part bytes, utiles)."""
    n = len(flux)
    sortes = np.array([f[0] for f in flux], dtype=np.uint8)
    mats = np.array([f[1] for f in flux], dtype=np.uint8)
    ctxs = np.array([f[2] for f in flux], dtype=np.uint8)
    prod = np.array([f[3] for f in flux], dtype=np.uint32)
    bufs = [np.frombuffer(bytes(f[4]), dtype=np.uint8).copy() for f in flux]
    lons = np.array([b.size for b in bufs], dtype=np.uint32)
    ptrs = (u8p * max(n, 1))(*[_p(b, u8p) for b in bufs])
    u = C.c_uint32()
    tot = lib().orc_assembler_partie(couche, expert, niveau, n_matrices, n, _p(sortes, u8p), _p(mats, u8p),
                                     _p(ctxs, u8p), _p(prod, u32p), ptrs, _p(lons, u32p), u8p(), 0, C.byref(u))
    out = np.zeros(tot, dtype=np.uint8)
    lib().orc_assembler_partie(couche, expert, niveau, n_matrices, n, _p(sortes, u8p), _p(mats, u8p), _p(ctxs, u8p),
                               _p(prod, u32p), ptrs, _p(lons, u32p), _p(out, u8p), tot, C.byref(u))
    return out.tobytes(), u.value


def lire_partie(octets: bytes):
    buf = np.frombuffer(octets, dtype=np.uint8).copy()
    p = Partie()
    if lib().orc_lire_partie(_p(buf, u8p), buf.size, C.byref(p)) != 0:
        return None
    return p


def coder_expert(blocs, biais, R, C_, freqs, couche=0, expert=0, canonique=True, N_delta=256, N_codes=256):
    """blocs: list (per matrix) of R*B*17 u8; biais: list of f32 arrays; freqs: list of (4,256) u16."""
    n = len(blocs)
    Ra = np.array(R, dtype=np.uint32)
    Ca = np.array(C_, dtype=np.uint32)
    bl = [np.ascontiguousarray(b, dtype=np.uint8) for b in blocs]
    bi = [np.ascontiguousarray(np.asarray(b, dtype=np.float32)).view(np.uint8) for b in biais]
    fr = [np.ascontiguousarray(f, dtype=np.uint16).reshape(-1) for f in freqs]
    pb = (u8p * n)(*[_p(a, u8p) for a in bl])
    pbi = (u8p * n)(*[_p(a, u8p) for a in bi])
    pf = (u16p * n)(*[_p(a, u16p) for a in fr])
    u = C.c_uint32()
    args = (couche, expert, n, _p(Ra, u32p), _p(Ca, u32p), pb, pbi, pf, int(canonique), N_delta, N_codes)
    tot = lib().orc_coder_expert(*args, u8p(), 0, C.byref(u))
    if tot == 0:
        raise ValueError("encoding refused")
    out = np.zeros(tot, dtype=np.uint8)
    lib().orc_coder_expert(*args, _p(out, u8p), tot, C.byref(u))
    return out.tobytes(), u.value


def decoder_matrice(partie: bytes, j: int, R: int, B: int, luts4: np.ndarray):
    buf = np.frombuffer(partie, dtype=np.uint8).copy()
    codes = np.zeros(16 * R * B, dtype=np.uint8)
    ech = np.zeros(R * B, dtype=np.uint8)
    bi = np.zeros(4 * R, dtype=np.uint8)
    bd, bc = Bilan(), Bilan()
    l4 = np.ascontiguousarray(luts4, dtype=np.uint32)
    r = lib().orc_decoder_matrice(_p(buf, u8p), buf.size, j, R, B, _p(l4, u32p), _p(codes, u8p), _p(ech, u8p),
                                  _p(bi, u8p), C.byref(bd), C.byref(bc))
    if r != 0:
        return None
    return codes, ech, bi.view(np.float32), bd, bc


def disposition_matrice(R: int, C_: int) -> Disposition:
    return lib().orc_disposition_matrice(R, C_)


def taille_emplacement(lignes, colonnes) -> int:
    a = np.array(lignes, dtype=np.uint32)
    b = np.array(colonnes, dtype=np.uint32)
    return lib().orc_taille_emplacement(_p(a, u32p), _p(b, u32p))


def disposition_j(lignes, colonnes, j) -> Disposition:
    a = np.array(lignes, dtype=np.uint32)
    b = np.array(colonnes, dtype=np.uint32)
    return lib().orc_disposition_j(_p(a, u32p), _p(b, u32p), j)


def decoder_expert(partie: bytes, luts: np.ndarray, lignes, colonnes):
    """Returns (slot bytes, ctl u32[4])."""
    buf = np.frombuffer(partie, dtype=np.uint8).copy()
    a = np.array(lignes, dtype=np.uint32)
    b = np.array(colonnes, dtype=np.uint32)
    te = taille_emplacement(lignes, colonnes)
    empl = np.zeros(te, dtype=np.uint8)
    ctl = np.zeros(4, dtype=np.uint32)
    lt = np.ascontiguousarray(luts, dtype=np.uint32)
    lib().orc_decoder_expert(_p(buf, u8p), buf.size, _p(lt, u32p), _p(a, u32p), _p(b, u32p), _p(empl, u8p),
                             _p(ctl, u32p))
    return empl, ctl


def gemv_mxfp4(matrice: np.ndarray, x: np.ndarray, R: int, C_: int) -> np.ndarray:
    m = np.ascontiguousarray(matrice, dtype=np.uint8)
    xx = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(R, dtype=np.float32)
    lib().orc_gemv_mxfp4(_p(m, u8p), _p(xx, f32p), _p(y, f32p), R, C_)
    return y


def gemv_mxfp4_f64(matrice: np.ndarray, x: np.ndarray, R: int, C_: int) -> np.ndarray:
    m = np.ascontiguousarray(matrice, dtype=np.uint8)
    xx = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(R, dtype=np.float64)
    lib().orc_gemv_mxfp4_f64(_p(m, u8p), _p(xx, f32p), _p(y, f64p), R, C_)
    return y


def gemv_f32(W: np.ndarray, x: np.ndarray, biais=None) -> np.ndarray:
    w = np.ascontiguousarray(W, dtype=np.float32)
    R, C_ = w.shape
    xx = np.ascontiguousarray(x, dtype=np.float32)
    b = np.ascontiguousarray(biais, dtype=np.float32) if biais is not None else None
    y = np.zeros(R, dtype=np.float32)
    lib().orc_gemv_f32(_p(w, f32p), _p(xx, f32p), _p(b, f32p) if b is not None else f32p(), _p(y, f32p), R, C_)
    return y


def swiglu_oai(g, u) -> np.ndarray:
    gg = np.ascontiguousarray(g, dtype=np.float32)
    uu = np.ascontiguousarray(u, dtype=np.float32)
    y = np.zeros(gg.size, dtype=np.float32)
    lib().orc_swiglu_oai(_p(gg, f32p), _p(uu, f32p), _p(y, f32p), gg.size)
    return y


def combiner(residu, sorties, pas, poids, n, d) -> np.ndarray:
    r = np.array(residu, dtype=np.float32)
    s = np.ascontiguousarray(sorties, dtype=np.float32)
    w = np.ascontiguousarray(poids, dtype=np.float32) if poids is not None else None
    lib().orc_combiner(_p(r, f32p), _p(s, f32p), pas, _p(w, f32p) if w is not None else f32p(), n, d)
    return r


def routeur_topk(logits, k):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.zeros(k, dtype=np.uint32)
    w = np.zeros(k, dtype=np.float32)
    lib().orc_routeur_topk(_p(lg, f32p), lg.size, k, _p(idx, u32p), _p(w, f32p))
    return idx, w


def routeur_topk_biais(logits, biais, k):
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    b = np.ascontiguousarray(biais, dtype=np.float32)
    assert b.size == lg.size
    idx = np.zeros(k, dtype=np.uint32)
    w = np.zeros(k, dtype=np.float32)
    lib().orc_routeur_topk_biais(_p(lg, f32p), _p(b, f32p), lg.size, k, _p(idx, u32p), _p(w, f32p))
    return idx, w


def synth_matrice(graine, couche, expert, cle, R, C_, avec_biais=True):
    nb = R * (C_ // 32)
    bl = np.zeros(17 * nb, dtype=np.uint8)
    bi = np.zeros(R, dtype=np.float32)
    lib().orc_synth_matrice(graine, couche, expert, cle, R, C_, _p(bl, u8p), _p(bi, f32p) if avec_biais else f32p())
    return bl, bi


def synth_normale_bf16(graine, cle1, cle2, n, sigma) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib().orc_synth_normale_bf16(graine, cle1, cle2, n, sigma, _p(out, f32p))
    return out


def empreinte64(octets: bytes) -> int:
    b = np.frombuffer(octets, dtype=np.uint8).copy() if len(octets) else np.zeros(1, dtype=np.uint8)
    return lib().orc_empreinte64(_p(b, u8p), len(octets))


def splitmix64_suite(graine: int, n: int):
    e = C.c_uint64(graine)
    return [lib().orc_splitmix64(C.byref(e)) for _ in range(n)]


def xorshift_suite(graine: int, n: int):
    e = C.c_uint64(graine)
    return [lib().orc_xorshift64s(C.byref(e)) for _ in range(n)]


# ------------------------------------------------------------------------ workload helpers

def blocs_vers_soa(blocs17: np.ndarray, R: int, C_: int, biais: np.ndarray, canonique: bool = True) -> np.ndarray:
    """One matrix in the SoA slot layout (abi.rs:76-88) from its 17-byte blocks (what the
    decoder must write). canonique folds nibble 8 to 0 (v1.2)."""
    nb = R * (C_ // 32)
    d = disposition_matrice(R, C_)
    out = np.zeros(d.pas, dtype=np.uint8)
    b = np.asarray(blocs17, dtype=np.uint8).reshape(nb, 17)
    qs = b[:, 1:].reshape(-1).copy()
    if canonique:
        lo = qs & 15
        hi = qs >> 4
        lo[lo == 8] = 0
        hi[hi == 8] = 0
        qs = (lo | (hi << 4)).astype(np.uint8)
    out[:16 * nb] = qs
    out[d.echelles:d.echelles + nb] = b[:, 0]
    out[d.biais:d.biais + 4 * R] = np.asarray(biais, dtype=np.float32).view(np.uint8)
    return out


# ---------------------------------------------------------------- forward pass around the experts

def f16_depuis_f32(v) -> np.ndarray:
    a = np.ascontiguousarray(v, dtype=np.float32).ravel()
    return np.array([lib().orc_f16_depuis_f32(float(x)) for x in a], dtype=np.uint16)


def f32_depuis_f16(h) -> np.ndarray:
    a = np.ascontiguousarray(h, dtype=np.uint16).ravel()
    return np.array([lib().orc_f32_depuis_f16(int(x)) for x in a], dtype=np.float32)


def gemv_q8_0(W: np.ndarray, x: np.ndarray, biais, R: int, C_: int) -> np.ndarray:
    w = np.ascontiguousarray(W, dtype=np.uint8)
    xx = np.ascontiguousarray(x, dtype=np.float32)
    b = np.ascontiguousarray(biais, dtype=np.float32) if biais is not None else None
    y = np.zeros(R, dtype=np.float32)
    lib().orc_gemv_q8_0(_p(w, u8p), _p(xx, f32p), _p(b, f32p) if b is not None else f32p(), _p(y, f32p), R, C_)
    return y


def ligne_q8_0(W: np.ndarray, ligne: int, C_: int) -> np.ndarray:
    w = np.ascontiguousarray(W, dtype=np.uint8)
    y = np.zeros(C_, dtype=np.float32)
    lib().orc_ligne_q8_0(_p(w, u8p), ligne, C_, _p(y, f32p))
    return y


def rmsnorm(x: np.ndarray, w: np.ndarray, n: int, lignes: int, eps: float) -> np.ndarray:
    xx = np.ascontiguousarray(x, dtype=np.float32)
    ww = np.ascontiguousarray(w, dtype=np.float32)
    y = np.zeros(n * lignes, dtype=np.float32)
    lib().orc_rmsnorm(_p(xx, f32p), _p(ww, f32p), _p(y, f32p), n, lignes, eps)
    return y


def inv_freq_yarn(p: ParamsRope, i: int):
    m, b, h = C.c_double(), C.c_double(), C.c_double()
    f = lib().orc_inv_freq_yarn(C.byref(p), i, C.byref(m), C.byref(b), C.byref(h))
    return f, m.value, b.value, h.value


def rope_yarn(q: np.ndarray, k: np.ndarray, tetes_q: int, tetes_k: int, position: int, p: ParamsRope):
    qq = np.array(q, dtype=np.float32)
    kk = np.array(k, dtype=np.float32)
    lib().orc_rope_yarn(_p(qq, f32p), _p(kk, f32p), tetes_q, tetes_k, position, C.byref(p))
    return qq, kk


def ecrire_kv(k, v, cache_k, cache_v, dkv: int, case_kv: int):
    kk = np.ascontiguousarray(k, dtype=np.float32)
    vv = np.ascontiguousarray(v, dtype=np.float32)
    ck = np.array(cache_k, dtype=np.uint16)
    cv = np.array(cache_v, dtype=np.uint16)
    lib().orc_ecrire_kv(_p(kk, f32p), _p(vv, f32p), _p(ck, u16p), _p(cv, u16p), dkv, case_kv)
    return ck, cv


def attention(q, cache_k, cache_v, puits, p: ParamsAttention) -> np.ndarray:
    qq = np.ascontiguousarray(q, dtype=np.float32)
    ck = np.ascontiguousarray(cache_k, dtype=np.uint16)
    cv = np.ascontiguousarray(cache_v, dtype=np.uint16)
    pu = np.ascontiguousarray(puits, dtype=np.float32)
    s = np.zeros(64 * p.tetes, dtype=np.float32)
    lib().orc_attention(_p(qq, f32p), _p(ck, u16p), _p(cv, u16p), _p(pu, f32p), _p(s, f32p), C.byref(p))
    return s


def argmax(v) -> int:
    vv = np.ascontiguousarray(v, dtype=np.float32)
    return int(lib().orc_argmax(_p(vv, f32p), vv.size))
