"""GPU parity of the batched prefill (trc_prefill_moe), through the C-ABI.

Each position's residual is checked against the reference's own chain run by the oracle for every
(position, slot) — gemv_mxfp4 gate and up, swiglu_oai, gemv_mxfp4 down, then the ordered combine
(trc-modele/src/lib.rs:688-710, passe.cuh:598-622) — and against the same computation in f64 from the
uncompressed weights: within 1e-5 * max|change| of both, per position (the fused path's GEMV
tolerance: gate and up multiply exact bf16 pieces of x, down exact bf16 pieces of act, so only the
fp32 accumulation order differs). Decoded weights are checked bit for bit by the other suites.
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle_ffi as O  # noqa: E402
from gpu_outils import dev, hote, vue, zeros  # noqa: E402
from troncons_amd import codeur, fusion  # noqa: E402
from troncons_amd import noyaux as K  # noqa: E402
from troncons_amd.noyaux import DimsExpert  # noqa: E402

TOL = 1e-5
GPT = DimsExpert.gpt_oss()


@pytest.fixture(scope="module")
def fz():
    return fusion.Fusion()


def _routage(graine, T, E, k, zipf=None):
    """k distinct experts per position (uniform or Zipf over the expert ranks) and softmax weights of
    seeded logits, computed in f64 and rounded once."""
    rng = np.random.default_rng(graine)
    idx = np.zeros((T, k), np.uint32)
    w = np.zeros((T, k), np.float32)
    p = None
    if zipf:
        p = 1.0 / np.arange(1, E + 1, dtype=np.float64) ** zipf
        p /= p.sum()
    for i in range(T):
        idx[i] = rng.choice(E, size=k, replace=False, p=p)
        lg = np.sort(rng.standard_normal(k))[::-1]
        ex = np.exp(lg - lg[0])
        w[i] = (ex / ex.sum()).astype(np.float32)
    return idx, w


def _slots(graine, E, dims):
    out = []
    for e in range(E):
        bl, bi = codeur.synth_expert(graine, 0, e, dims)
        out.append([O.blocs_vers_soa(bl[j], dims.lignes[j], dims.colonnes[j], bi[j], canonique=True)
                    for j in range(3)])
    return out


def _mlp(sl, x, dims):
    R, C = dims.lignes[0], dims.colonnes[0]
    g = O.gemv_mxfp4(sl[0], x, R, C)
    u = O.gemv_mxfp4(sl[1], x, R, C)
    s = O.gemv_mxfp4(sl[2], O.swiglu_oai(g, u), dims.lignes[2], dims.colonnes[2])
    g64 = O.gemv_mxfp4_f64(sl[0], x, R, C)
    u64 = O.gemv_mxfp4_f64(sl[1], x, R, C)
    gg = np.minimum(g64, 7.0)
    uu = np.clip(u64, -7.0, 7.0)
    a64 = gg / (1.0 + np.exp(-1.702 * gg)) * (uu + 1.0)
    s64 = O.gemv_mxfp4_f64(sl[2], a64.astype(np.float32), dims.lignes[2], dims.colonnes[2])
    return s, s64


class Couche:
    """A synthetic layer mounted on the device (parts, directory, LUTs)."""

    def __init__(self, fz, graine, E, dims, N):
        self.c = codeur.CoucheSynthetique(graine, 0, E, dims, N_delta=N[0], N_codes=N[1])
        freqs = self.c.freqs()
        self.luts = dev(O.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)]))
        self.parts = [dev(self.c.partie(e)) for e in range(E)]
        self.table = dev(np.array([p.data_ptr() for p in self.parts], np.uint64))
        self.rep = zeros(fusion.taille_repertoire(E))
        ctl = zeros(16)
        fz.monter_couche(vue(self.table), E, dims, vue(self.rep), vue(ctl))
        assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]


def _lancer(fz, couche, E, dims, x, idx, w, residu0, N, pieces=None):
    T, k = idx.shape
    xd, idd, wd, res = dev(x), dev(idx), dev(w), dev(residu0)
    ctl = zeros(16)
    tr = zeros(fusion.taille_travail_prefill(dims, E, T, k, N[1]))
    print(f"prefill: T={T} k={k} E={E} dims={list(dims.lignes)}x{list(dims.colonnes)} N={N}", flush=True)
    fz.prefill_moe(vue(couche.rep), E, vue(couche.luts), dims, vue(xd), T, vue(idd), vue(wd), k, vue(res), vue(ctl),
                   vue(tr), *N)
    if pieces is not None:  # the workspace starts with the pieces used by x and by act
        pieces.extend(int(v) for v in hote(tr, np.uint32)[:2])
    return hote(res, np.float32).reshape(T, -1), hote(ctl, np.uint32)


def _verifier(got, residu0, x, idx, w, slots, dims, valides=None):
    T, k = idx.shape
    D = dims.lignes[2]
    for i in range(T):
        if valides is not None and not valides[i]:
            assert (got[i] == residu0[i]).all()
            continue
        s, s64 = zip(*[_mlp(slots[int(idx[i, q])], x[i], dims) for q in range(k)])
        ref = O.combiner(residu0[i], np.concatenate(s), D, w[i], k, D)
        ref64 = residu0[i].astype(np.float64) + sum(float(w[i, q]) * s64[q] for q in range(k))
        d = ref - residu0[i]
        assert np.abs(got[i] - ref).max() <= TOL * np.abs(d).max(), i
        assert np.abs(got[i] - ref64).max() <= TOL * np.abs(ref64 - residu0[i]).max(), i


@pytest.mark.parametrize("N", [(8, 8), (4, 16), (16, 3)])
def test_prefill_small_layer_zipf_routing(fz, N):
    """6 experts, 40 positions, Zipf routing (some experts take more than 16 positions: several
    MFMA column tiles), 256-wide matrices."""
    E, T, k = 6, 40, 4
    dims = DimsExpert.de([256, 256, 256], [256, 256, 256])
    couche = Couche(fz, 31, E, dims, N)
    idx, w = _routage(32, T, E, k, zipf=1.1)
    x = np.stack([O.synth_normale_bf16(33, 4, i, 256, 1.0) for i in range(T)])
    residu0 = np.stack([O.synth_normale_bf16(33, 5, i, 256, 0.5) for i in range(T)])
    got, ctl = _lancer(fz, couche, E, dims, x, idx, w, residu0, N)
    assert list(ctl) == [0, 0, 0, 0]
    _verifier(got, residu0, x, idx, w, _slots(31, E, dims), dims)
    couche.c.liberer()


@pytest.mark.parametrize("N", [(8, 8), (1, 16)])
def test_prefill_ragged_blocks(fz, N):
    """Rows of 9 and 11 blocks (padded to 12 for the 4-block MFMA step), 288-wide layer; with
    N = (1, 16) the experts go through their slots (gate and up in bands of 32 rows: 11 and 9
    bands)."""
    E, T, k = 5, 21, 3
    dims = DimsExpert.de([352, 352, 288], [288, 288, 352])
    couche = Couche(fz, 41, E, dims, N)
    idx, w = _routage(42, T, E, k)
    x = np.stack([O.synth_normale_bf16(43, 4, i, 288, 1.0) for i in range(T)])
    residu0 = np.zeros((T, 288), np.float32)
    got, ctl = _lancer(fz, couche, E, dims, x, idx, w, residu0, N)
    assert list(ctl) == [0, 0, 0, 0]
    _verifier(got, residu0, x, idx, w, _slots(41, E, dims), dims)
    couche.c.liberer()


@pytest.mark.parametrize("N", [(8, 8), (1, 16)])
@pytest.mark.parametrize("bits", [24, 16])
def test_prefill_f32_activations(fz, bits, N):
    """x with full f32 significands (gate and up then take three bf16 pieces of x) or with 16-bit ones
    (two pieces), on the ragged layer and on the small one; N = (1, 16) takes the slot path."""
    for graine, dims, E, T, k in [(61, DimsExpert.de([352, 352, 288], [288, 288, 352]), 5, 21, 3),
                                  (71, DimsExpert.de([256, 256, 256], [256, 256, 256]), 6, 40, 4)]:
        C = dims.colonnes[0]
        couche = Couche(fz, graine, E, dims, N)
        idx, w = _routage(graine + 1, T, E, k, zipf=1.1)
        rng = np.random.default_rng(graine + 2)
        x = rng.standard_normal((T, C)).astype(np.float32)
        x *= np.exp2(rng.integers(-6, 7, size=(T, C))).astype(np.float32)  # a wide range within each block
        if bits == 16:
            x = (x.view(np.uint32) & np.uint32(0xFFFFFF00)).view(np.float32)
        residu0 = np.zeros((T, dims.lignes[2]), np.float32)
        pieces = []
        got, ctl = _lancer(fz, couche, E, dims, x, idx, w, residu0, N, pieces)
        assert list(ctl) == [0, 0, 0, 0]
        assert pieces[0] == (3 if bits == 24 else 2), pieces
        _verifier(got, residu0, x, idx, w, _slots(graine, E, dims), dims)
        couche.c.liberer()


def test_prefill_wide_rows(fz):
    """4096-wide matrices: the band is 32 rows (two MFMA row tiles), so the passes over one and two
    column tiles run with nrt = 2; Zipf routing gives the first expert more than 16 pairs."""
    E, T, k, N = 3, 20, 2, (1, 16)
    dims = DimsExpert.de([4096, 4096, 4096], [4096, 4096, 4096])
    couche = Couche(fz, 81, E, dims, N)
    idx, w = _routage(82, T, E, k, zipf=1.1)
    assert np.bincount(idx.reshape(-1), minlength=E).max() > 16
    x = np.stack([O.synth_normale_bf16(83, 4, i, 4096, 1.0) for i in range(T)])
    residu0 = np.zeros((T, 4096), np.float32)
    got, ctl = _lancer(fz, couche, E, dims, x, idx, w, residu0, N)
    assert list(ctl) == [0, 0, 0, 0]
    _verifier(got, residu0, x, idx, w, _slots(81, E, dims), dims)
    couche.c.liberer()


def test_prefill_band_heights(fz):
    """Band heights by row width: gate and up are 3072 wide (96 blocks a row: 64-row bands, four
    MFMA row tiles), down is 256 wide (8 blocks: 80-row bands, five row tiles) over 3072 rows, so its
    last band holds 32 rows and 48 padding rows; Zipf routing gives one expert more than 32 pairs,
    so the paired and single column-tile passes both run at both heights."""
    E, T, k, N = 3, 40, 2, (1, 16)
    dims = DimsExpert.de([256, 256, 3072], [3072, 3072, 256])
    couche = Couche(fz, 91, E, dims, N)
    idx, w = _routage(92, T, E, k, zipf=1.1)
    assert np.bincount(idx.reshape(-1), minlength=E).max() > 32
    x = np.stack([O.synth_normale_bf16(93, 4, i, 3072, 1.0) for i in range(T)])
    residu0 = np.stack([O.synth_normale_bf16(94, 4, i, 3072, 0.5) for i in range(T)])
    got, ctl = _lancer(fz, couche, E, dims, x, idx, w, residu0, N)
    assert list(ctl) == [0, 0, 0, 0]
    _verifier(got, residu0, x, idx, w, _slots(91, E, dims), dims)
    couche.c.liberer()


def test_prefill_gpt_oss_shape(fz):
    """Config-5 shape family: 2880 x 2880 gpt-oss experts, N = 16 / 4, 16 positions over 8 experts
    with Zipf routing; also determinism (a second call gives the same bits)."""
    E, T, k, N = 8, 16, 4, (4, 16)
    couche = Couche(fz, 51, E, GPT, N)
    idx, w = _routage(52, T, E, k, zipf=1.1)
    x = np.stack([O.synth_normale_bf16(53, 4, i, 2880, 1.0) for i in range(T)])
    residu0 = np.zeros((T, 2880), np.float32)
    pieces = []
    got, ctl = _lancer(fz, couche, E, GPT, x, idx, w, residu0, N, pieces)
    assert list(ctl) == [0, 0, 0, 0]
    assert pieces[0] == 1, pieces  # bf16 activations: one bf16 piece of x
    got2, _ = _lancer(fz, couche, E, GPT, x, idx, w, residu0, N)
    assert (got == got2).all()
    _verifier(got, residu0, x, idx, w, _slots(51, E, GPT), GPT)
    couche.c.liberer()


def test_prefill_bad_indices_counted_and_skipped(fz):
    """Indices >= experts are format errors: counted once each, their positions untouched; the other
    positions are still right."""
    E, T, k, N = 4, 12, 2, (8, 8)
    dims = DimsExpert.de([256, 256, 256], [256, 256, 256])
    couche = Couche(fz, 61, E, dims, N)
    idx, w = _routage(62, T, E, k)
    idx[3, 1] = E
    idx[7, 0] = 1000
    x = np.stack([O.synth_normale_bf16(63, 4, i, 256, 1.0) for i in range(T)])
    residu0 = np.stack([O.synth_normale_bf16(63, 5, i, 256, 0.5) for i in range(T)])
    got, ctl = _lancer(fz, couche, E, dims, x, idx, w, residu0, N)
    assert ctl[1] == 2 and ctl[0] == 0 and ctl[2] == 0 and ctl[3] == 0
    valides = [i not in (3, 7) for i in range(T)]
    _verifier(got, residu0, x, idx, w, _slots(61, E, dims), dims, valides)
    couche.c.liberer()


def _decaler_debut_delta(partie: np.ndarray, j: int, t: int) -> np.ndarray:
    """The part with the first word of DELTA tile t of matrix j moved one word later, kept inside
    [start[t-1], start[t+1]] (the starts stay monotonic; only the tile boundary is wrong)."""
    p = partie.copy()
    n = int.from_bytes(p[10:12].tobytes(), "little")
    (d,) = [64 + 16 * i for i in range(n) if p[64 + 16 * i] == 3 and p[64 + 16 * i + 1] == j]  # DELTA = kind 3
    dec = int.from_bytes(p[d + 4:d + 8].tobytes(), "little")
    T = int.from_bytes(p[dec + 8:dec + 12].tobytes(), "little")
    debuts = p[dec + 16:dec + 16 + 4 * T].view(np.uint32)
    assert 0 < t < T - 1 and debuts[t] + 1 <= debuts[t + 1]
    debuts[t] += 1
    return p


def test_prefill_delta_interior_tile_start_counted(fz):
    """The prefill's DELTA pass decodes runs of consecutive tiles through one word ring (about 5
    tiles per half-wavefront for 8 gpt-oss experts at N_delta = 1). A tile start moved inside a run
    leaves the decoded bytes intact, but the reference flags the tile before it (its words do not
    end on the next tile's first word, rans.rs:442-448): the pass must count it in the pointer word."""
    E, T, k, N = 8, 4, 4, (1, 8)
    couche = Couche(fz, 101, E, GPT, N)
    idx = np.array([[0, 1, 2, 3], [4, 5, 6, 0], [7, 0, 1, 2], [0, 3, 5, 7]], np.uint32)
    w = np.full((T, k), 0.25, np.float32)
    x = np.stack([O.synth_normale_bf16(103, 4, i, 2880, 1.0) for i in range(T)])
    residu0 = np.zeros((T, 2880), np.float32)
    _, ctl = _lancer(fz, couche, E, GPT, x, idx, w, residu0, N)
    assert list(ctl) == [0, 0, 0, 0]
    # tile 1 of expert 0's gate DELTA stream: the second tile of the first run
    abime = _decaler_debut_delta(couche.c.partie(0), 0, 1)
    couche.parts[0].copy_(torch.from_numpy(abime))
    _, ctl = _lancer(fz, couche, E, GPT, x, idx, w, residu0, N)
    assert ctl[2] >= 1 and ctl[1] == 0, list(ctl)
    couche.c.liberer()


def test_prefill_reference_tile_lengths_gpt_oss_shape(fz):
    """Streams written with the reference encoder's tile lengths (N = 256 for DELTA and CODES_CTX,
    rans.rs:32): the chosen experts are decoded once into slots, the bands read them. 8 gpt-oss
    experts, 16 positions with Zipf routing: every position within 1e-5 of the oracle chain and of
    f64; a flipped bit in a chosen expert's CODES_CTX stream is counted."""
    E, T, k, N = 8, 16, 4, (256, 256)
    couche = Couche(fz, 111, E, GPT, N)
    idx, w = _routage(112, T, E, k, zipf=1.1)
    x = np.stack([O.synth_normale_bf16(113, 4, i, 2880, 1.0) for i in range(T)])
    residu0 = np.stack([O.synth_normale_bf16(113, 5, i, 2880, 0.5) for i in range(T)])
    got, ctl = _lancer(fz, couche, E, GPT, x, idx, w, residu0, N)
    assert list(ctl) == [0, 0, 0, 0]
    _verifier(got, residu0, x, idx, w, _slots(111, E, GPT), GPT)
    # a flipped bit in the middle of expert idx[0, 0]'s up CODES_CTX stream
    e0 = int(idx[0, 0])
    p = couche.c.partie(e0)
    n = int.from_bytes(p[10:12].tobytes(), "little")
    (d,) = [64 + 16 * i for i in range(n) if p[64 + 16 * i] == 4 and p[64 + 16 * i + 1] == 1]  # CODES_CTX = kind 4
    dec = int.from_bytes(p[d + 4:d + 8].tobytes(), "little")
    lon = int.from_bytes(p[d + 8:d + 12].tobytes(), "little")
    p[dec + lon // 2] ^= 0x10
    couche.parts[e0].copy_(torch.from_numpy(p))
    _, ctl = _lancer(fz, couche, E, GPT, x, idx, w, residu0, N)
    assert ctl[0] + ctl[2] > 0 and ctl[1] == 0, list(ctl)
    couche.c.liberer()


@pytest.mark.parametrize("N", [(1, 16), (2, 16), (2, 32)])
def test_prefill_delta_in_codes_gpt_oss_shape(fz, N):
    """Tile lengths whose DELTA the CODES pass decodes itself (16 with DELTA tiles of 1 or 2, 32 with
    2): the chosen experts are decoded into slots by one launch that decodes each tile's DELTA with
    it, the bands read the slots. 8 gpt-oss experts, 16 positions with Zipf routing, against the
    oracle chain and f64; a flipped bit in a chosen expert's DELTA stream is counted."""
    E, T, k = 8, 16, 4
    couche = Couche(fz, 121, E, GPT, N)
    idx, w = _routage(122, T, E, k, zipf=1.1)
    x = np.stack([O.synth_normale_bf16(123, 4, i, 2880, 1.0) for i in range(T)])
    residu0 = np.stack([O.synth_normale_bf16(123, 5, i, 2880, 0.5) for i in range(T)])
    got, ctl = _lancer(fz, couche, E, GPT, x, idx, w, residu0, N)
    assert list(ctl) == [0, 0, 0, 0]
    _verifier(got, residu0, x, idx, w, _slots(121, E, GPT), GPT)
    # a flipped bit in the middle of expert idx[0, 0]'s down DELTA stream
    e0 = int(idx[0, 0])
    p = couche.c.partie(e0)
    n = int.from_bytes(p[10:12].tobytes(), "little")
    (d,) = [64 + 16 * i for i in range(n) if p[64 + 16 * i] == 3 and p[64 + 16 * i + 1] == 2]  # DELTA = kind 3
    dec = int.from_bytes(p[d + 4:d + 8].tobytes(), "little")
    lon = int.from_bytes(p[d + 8:d + 12].tobytes(), "little")
    p[dec + lon // 2] ^= 0x10
    couche.parts[e0].copy_(torch.from_numpy(p))
    _, ctl = _lancer(fz, couche, E, GPT, x, idx, w, residu0, N)
    assert ctl[0] + ctl[2] > 0 and ctl[1] == 0, list(ctl)
    couche.c.liberer()


def _al(n):
    return (n + 255) // 256 * 256


@pytest.mark.parametrize("N", [(1, 16), (2, 16), (2, 32), ((2, 2, 1), (32, 32, 16)), (256, 256)])
def test_prefill_slots_bit_exact(fz, N):
    """The slot decoders' output itself, byte for byte: after a prefill whose routing chooses every
    expert, each expert's slot in the workspace holds exactly the code bytes and E8M0 scales of the
    oracle's canonical SoA slot (the reference decoder's output, -0 folded into +0). Tiles whose
    DELTA the CODES pass decodes (16/1, 16/2, 32/2, the bench's per-matrix encoding: the decode
    step's tile machinery) and the reference encoder's 256/256 (the generic slot decoders). The
    slots follow the piece counters, the per-expert counts and starts and the pair list, each
    256-byte aligned; the bias area of a slot is not written by the decoders and is not compared."""
    E, T, k = 4, 8, 4
    appel = tuple(n if isinstance(n, int) else n[2] for n in N)  # the call takes the down matrix's
    couche = Couche(fz, 131, E, GPT, N)
    idx = np.stack([np.random.default_rng(132 + i).permutation(E) for i in range(T)]).astype(np.uint32)
    w = np.full((T, k), 0.25, np.float32)
    x = np.stack([O.synth_normale_bf16(133, 4, i, 2880, 1.0) for i in range(T)])
    xd, idd, wd, res = dev(x), dev(idx), dev(w), dev(np.zeros((T, 2880), np.float32))
    ctl = zeros(16)
    tr = zeros(fusion.taille_travail_prefill(GPT, E, T, k, appel[1]))
    print(f"prefill slots: E={E} T={T} N={N}", flush=True)
    fz.prefill_moe(vue(couche.rep), E, vue(couche.luts), GPT, vue(xd), T, vue(idd), vue(wd), k, vue(res), vue(ctl),
                   vue(tr), *appel)
    assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]
    ws = hote(tr)
    pas = K.taille_emplacement(GPT)
    o = _al(16) + 2 * _al(4 * E) + _al(4 * T * k)
    attendus = _slots(131, E, GPT)
    for e in range(E):
        slot = ws[o + e * pas:o + (e + 1) * pas]
        for j in range(3):
            d = O.disposition_j(list(GPT.lignes), list(GPT.colonnes), j)
            nb = GPT.lignes[j] * (GPT.colonnes[j] // 32)
            a = attendus[e][j]
            # codes at the matrix's base, scales at its echelles offset (both in the oracle's layout)
            assert (slot[d.base:d.base + 16 * nb] == a[:16 * nb]).all(), (e, j, "codes")
            assert (slot[d.base + d.echelles:d.base + d.echelles + nb] == a[d.echelles:d.echelles + nb]).all(), \
                (e, j, "scales")
    couche.c.liberer()
