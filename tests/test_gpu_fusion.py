"""GPU parity of the fused path (decode in registers + GEMV / SwiGLU / combine) against the CPU
oracle, through the C-ABI.

Tolerance (stated, the reference's own GEMV threshold, decisions/ARCHITECTURE.md §5.6 table):
every output within 1e-5 * max|y| of the f64 computation from the uncompressed weights, and of the
reference's f32 operation order. On the integer-exact fixture (scales in [117,123], x in {-2,-1,1,2},
tests/carte.rs:1-10) every partial sum is exact in f32, so the fused GEMV must match bit for bit
whatever its summation order. Decoded-byte exactness is checked through the control words and
that exact GEMV.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle_ffi as O  # noqa: E402
from gpu_outils import Expert, dev, hote, vue, zeros  # noqa: E402
from troncons_amd import codeur, fusion  # noqa: E402
from troncons_amd import noyaux as K  # noqa: E402
from troncons_amd.noyaux import DimsExpert  # noqa: E402

GPT = DimsExpert.gpt_oss()
TOL = 1e-5


@pytest.fixture(scope="module")
def fz():
    assert torch.cuda.is_available()
    return fusion.Fusion()


def _gemv(fz, partie, luts, j, R, C, x, n_delta, n_codes):
    p, l, xd = dev(partie), dev(luts), dev(x)
    y = zeros(4 * R)
    ctl = zeros(16)
    tr = zeros(fusion.taille_travail_gemv(R, C, n_codes))
    fz.gemv_fusionnee(vue(p), j, vue(l), R, C, vue(xd), vue(y), vue(ctl), vue(tr), n_delta, n_codes)
    return hote(y, np.float32), hote(ctl, np.uint32)


def _slot_j(ex, j):
    d = O.disposition_j([2880] * 3, [2880] * 3, j)
    return ex.attendu[d.base:d.base + d.pas]


@pytest.mark.parametrize("N", [(256, 256), (32, 32), (8, 16), (4, 1), (1, 16), (2, 16), (2, 32)])
def test_fused_gemv_one_matrix_config1(fz, N):
    ex = Expert(2026, GPT, N_delta=N[0], N_codes=N[1])
    x = O.synth_normale_bf16(2026, 1, 0, 2880, 1.0)
    for j in (2, 0):
        y, ctl = _gemv(fz, ex.partie, ex.luts, j, 2880, 2880, x, *N)
        assert list(ctl) == [0, 0, 0, 0]
        y64 = O.gemv_mxfp4_f64(_slot_j(ex, j), x, 2880, 2880)
        assert np.abs(y - y64).max() <= TOL * np.abs(y64).max()
        yref = O.gemv_mxfp4(_slot_j(ex, j), x, 2880, 2880)
        assert np.abs(y - yref).max() <= TOL * np.abs(y64).max()
        y2, _ = _gemv(fz, ex.partie, ex.luts, j, 2880, 2880, x, *N)
        assert (y.view(np.uint32) == y2.view(np.uint32)).all(), "fused GEMV not deterministic"


def _expert_exact(seed, dims):
    rng = np.random.default_rng(seed)
    blocs, biais = [], []
    for j in range(3):
        r, c = dims.lignes[j], dims.colonnes[j]
        nb = r * (c // 32)
        e = rng.integers(117, 124, nb).astype(np.uint8)
        u = rng.integers(0, 100, (nb, 32))
        mag = np.where(u < 40, u % 2, np.where(u < 80, 2 + u % 3, 5 + u % 3))
        code = mag | (rng.integers(0, 2, (nb, 32)) << 3)
        bl = np.zeros((nb, 17), np.uint8)
        bl[:, 0] = e
        bl[:, 1:] = (code[:, :16] | (code[:, 16:] << 4)).astype(np.uint8)
        blocs.append(bl.reshape(-1))
        biais.append(((rng.integers(0, 2001, r) - 1000) / 2048.0).astype(np.float32))
    return blocs, biais


@pytest.mark.parametrize("N", [(256, 256), (16, 32), (3, 7), (1, 16), (2, 16), (2, 32)])
def test_fused_gemv_bit_exact_on_integer_fixture(fz, N):
    dims = GPT
    blocs, biais = _expert_exact(7, dims)
    freqs = [codeur.tables([blocs[j]], 2880, 90) for j in range(3)]
    partie, _ = codeur.partie(blocs, biais, freqs, dims, N_delta=N[0], N_codes=N[1])
    luts = O.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)])
    # no zero in x: every decoded nibble reaches the sum, so a wrong one shows in its row
    x = np.random.default_rng(11).choice(np.array([-2.0, -1.0, 1.0, 2.0], np.float32), 2880)
    for j in range(3):
        y, ctl = _gemv(fz, partie, luts, j, 2880, 2880, x, *N)
        assert list(ctl) == [0, 0, 0, 0]
        slot = O.blocs_vers_soa(blocs[j], 2880, 2880, biais[j], canonique=True)
        y64 = O.gemv_mxfp4_f64(slot, x, 2880, 2880).astype(np.float32)
        assert (y.view(np.uint32) == y64.view(np.uint32)).all()


@pytest.mark.parametrize("N", [(1, 16), (2, 32)])
def test_fused_gemv_scales_outside_the_folded_range(fz, N):
    """Tiles whose exponents leave [64, 191] take the ldexp form instead of the scale folded into the
    conversion: rows 0-999 have e in [192, 200], rows 1000-1999 in [40, 63], the rest in [119, 125]
    (the fold), with tiles straddling the bands; each band within 1e-5 * its max|y| of f64."""
    dims = GPT
    rng = np.random.default_rng(13)
    blocs, biais = [], []
    for j in range(3):
        r, c = dims.lignes[j], dims.colonnes[j]
        nb = r * (c // 32)
        ligne = np.repeat(np.arange(r), c // 32)
        e = np.where(ligne < 1000, rng.integers(192, 201, nb),
                     np.where(ligne < 2000, rng.integers(40, 64, nb), rng.integers(119, 126, nb))).astype(np.uint8)
        bl = np.zeros((nb, 17), np.uint8)
        bl[:, 0] = e
        bl[:, 1:] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
        blocs.append(bl.reshape(-1))
        biais.append(np.zeros(r, np.float32))
    freqs = [codeur.tables([blocs[j]], 2880, 90) for j in range(3)]
    partie, _ = codeur.partie(blocs, biais, freqs, dims, N_delta=N[0], N_codes=N[1])
    luts = O.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)])
    x = O.synth_normale_bf16(13, 1, 0, 2880, 1.0)
    for j in (0, 2):
        y, ctl = _gemv(fz, partie, luts, j, 2880, 2880, x, *N)
        assert list(ctl) == [0, 0, 0, 0]
        slot = O.blocs_vers_soa(blocs[j], 2880, 2880, biais[j], canonique=True)
        y64 = O.gemv_mxfp4_f64(slot, x, 2880, 2880)
        for a, b in ((0, 1000), (1000, 2000), (2000, 2880)):
            assert np.abs(y[a:b] - y64[a:b]).max() <= TOL * np.abs(y64[a:b]).max(), (j, a)


@pytest.mark.parametrize("N", [(2, 3), (1, 16), (2, 16), (2, 32)])
def test_fused_gemv_small_shapes_and_break(fz, N):
    dims = DimsExpert.de([300, 300, 257], [256, 256, 320])
    ex = Expert(5, dims, N_delta=N[0], N_codes=N[1])
    for j in range(3):
        R, C = dims.lignes[j], dims.colonnes[j]
        x = O.synth_normale_bf16(5, 2, j, C, 1.0)
        y, ctl = _gemv(fz, ex.partie, ex.luts, j, R, C, x, *N)
        assert list(ctl) == [0, 0, 0, 0]
        d = O.disposition_j(list(dims.lignes), list(dims.colonnes), j)
        y64 = O.gemv_mxfp4_f64(ex.attendu[d.base:d.base + d.pas], x, R, C)
        assert np.abs(y - y64).max() <= TOL * np.abs(y64).max()
    # break: a flipped bit in CODES_CTX of matrix 1 is seen by the control words
    p = bytearray(ex.partie)
    e = 64 + 16 * 7
    dec = int.from_bytes(p[e + 4:e + 8], "little")
    lon = int.from_bytes(p[e + 8:e + 12], "little")
    p[dec + lon // 2] ^= 0x10
    _, ctl = _gemv(fz, bytes(p), ex.luts, 1, 300, 256, O.synth_normale_bf16(5, 2, 1, 256, 1.0), *N)
    assert ctl[0] > 0
    # a flipped bit in the DELTA stream of matrix 1 (its descriptor is 6)
    p = bytearray(ex.partie)
    e = 64 + 16 * 6
    dec = int.from_bytes(p[e + 4:e + 8], "little")
    lon = int.from_bytes(p[e + 8:e + 12], "little")
    p[dec + lon - 8] ^= 0x21
    _, ctl = _gemv(fz, bytes(p), ex.luts, 1, 300, 256, O.synth_normale_bf16(5, 2, 1, 256, 1.0), *N)
    assert ctl[0] + ctl[2] > 0
    p = bytearray(ex.partie)
    p[0] ^= 0xFF
    _, ctl = _gemv(fz, bytes(p), ex.luts, 1, 300, 256, O.synth_normale_bf16(5, 2, 1, 256, 1.0), *N)
    assert ctl[1] > 0


def test_fused_gemv_wide_rows(fz):
    """Rows wider than the LDS copy of x (3328 > 3072 columns) take the device-memory x variant."""
    dims = DimsExpert.de([48, 48, 64], [3328, 3328, 256])
    ex = Expert(9, dims, N_delta=3, N_codes=5)
    for j in (0, 2):
        R, C = dims.lignes[j], dims.colonnes[j]
        x = O.synth_normale_bf16(9, 2, j, C, 1.0)
        y, ctl = _gemv(fz, ex.partie, ex.luts, j, R, C, x, 3, 5)
        assert list(ctl) == [0, 0, 0, 0]
        d = O.disposition_j(list(dims.lignes), list(dims.colonnes), j)
        y64 = O.gemv_mxfp4_f64(ex.attendu[d.base:d.base + d.pas], x, R, C)
        assert np.abs(y - y64).max() <= TOL * np.abs(y64).max()


def _mlp_oracle(ex, x, dims):
    """The reference chain in its own f32 order (gemv x2, swiglu_oai, gemv) and in f64."""
    R, C = dims.lignes[0], dims.colonnes[0]
    sl = [ex.attendu[O.disposition_j(list(dims.lignes), list(dims.colonnes), j).base:][
          :O.disposition_j(list(dims.lignes), list(dims.colonnes), j).pas] for j in range(3)]
    g = O.gemv_mxfp4(sl[0], x, R, C)
    u = O.gemv_mxfp4(sl[1], x, R, C)
    a = O.swiglu_oai(g, u)
    s = O.gemv_mxfp4(sl[2], a, dims.lignes[2], dims.colonnes[2])
    g64 = O.gemv_mxfp4_f64(sl[0], x, R, C)
    u64 = O.gemv_mxfp4_f64(sl[1], x, R, C)
    gg = np.minimum(g64, 7.0)
    uu = np.clip(u64, -7.0, 7.0)
    a64 = gg / (1.0 + np.exp(-1.702 * gg)) * (uu + 1.0)
    s64 = O.gemv_mxfp4_f64(sl[2], a64.astype(np.float32), dims.lignes[2], dims.colonnes[2])
    return s, s64


@pytest.mark.parametrize("N", [(256, 256), (32, 32), (8, 16), (1, 16), (2, 16), (2, 32)])
def test_fused_expert_config2(fz, N):
    ex = Expert(2027, GPT, N_delta=N[0], N_codes=N[1])
    x = O.synth_normale_bf16(2027, 1, 0, 2880, 1.0)
    p, l, xd = dev(ex.partie), dev(ex.luts), dev(x)
    s = zeros(4 * 2880)
    ctl = zeros(16)
    tr = zeros(fusion.taille_travail_expert(GPT, N[1]))
    fz.expert_fusionne(vue(p), vue(l), GPT, vue(xd), vue(s), vue(ctl), vue(tr), *N)
    got = hote(s, np.float32)
    assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]
    s_ref, s64 = _mlp_oracle(ex, x, GPT)
    assert np.abs(got - s_ref).max() <= TOL * np.abs(s_ref).max()
    assert np.abs(got - s64).max() <= TOL * np.abs(s64).max()


@pytest.mark.parametrize("N", [(16, 32), (1, 16), (2, 16), ((2, 2, 1), (32, 32, 16))])
def test_fused_moe_layer_config3(fz, N):
    """N: (N_delta, N_codes), one value for the three matrices or one per matrix (the bench's
    gate/up at 2/32, down at 1/16); the layer step is called with the down matrix's."""
    E, k = 12, 4
    couche = codeur.CoucheSynthetique(2028, 0, E, GPT, N_delta=N[0], N_codes=N[1])
    N = tuple(n if isinstance(n, int) else n[2] for n in N)
    freqs = couche.freqs()
    luts = O.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)])
    parts = [dev(couche.partie(e)) for e in range(E)]
    table = dev(np.array([p.data_ptr() for p in parts], np.uint64))
    rep, ctl0 = zeros(fusion.taille_repertoire(E)), zeros(16)
    fz.monter_couche(vue(table), E, GPT, vue(rep), vue(ctl0))
    assert list(hote(ctl0, np.uint32)) == [0, 0, 0, 0]
    routeur = np.stack([O.synth_normale_bf16(2028, 3, e, 2880, 0.02) for e in range(E)])
    r16 = (routeur.view(np.uint32) >> 16).astype(np.uint16)
    x = O.synth_normale_bf16(2028, 4, 0, 2880, 1.0)
    residu0 = np.zeros(2880, np.float32)
    l, rd, xd, res = dev(luts), dev(r16), dev(x), dev(residu0)
    idx, w, ctl = zeros(32), zeros(32), zeros(16)
    tr = zeros(fusion.taille_travail_couche(GPT, E, k, N[1]))
    fz.couche_moe(vue(rep), E, vue(l), GPT, vue(rd), None, vue(xd), k, vue(res), vue(idx), vue(w), vue(ctl),
                  vue(tr), *N)
    got = hote(res, np.float32)
    assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]
    logits = O.gemv_f32(routeur, x)
    oi, ow = O.routeur_topk(logits, k)
    gi, gw = hote(idx, np.uint32)[:k], hote(w, np.float32)[:k]
    assert (gi == oi).all() and np.abs(gw - ow).max() <= 1e-6
    sorties = []
    sorties64 = []
    for e in oi:
        bl, bi = codeur.synth_expert(2028, 0, int(e), GPT)
        ex = type("E", (), {})()
        ex.attendu = np.concatenate([O.blocs_vers_soa(bl[j], 2880, 2880, bi[j], canonique=True) for j in range(3)])
        s, s64 = _mlp_oracle(ex, x, GPT)
        sorties.append(s)
        sorties64.append(s64)
    ref = O.combiner(residu0, np.concatenate(sorties), 2880, ow, k, 2880)
    ref64 = sum(float(ow[i]) * sorties64[i] for i in range(k))
    assert np.abs(got - ref).max() <= TOL * np.abs(ref).max()
    assert np.abs(got - ref64).max() <= TOL * np.abs(ref64).max()
    couche.liberer()


def _couche_oracle(graine, E, k, x, avant, routeur):
    """The reference layer step on the CPU: router logits, top-k, each chosen expert's MLP in the
    reference's f32 order, the ordered combine into `avant`; also the f64 sum of the products."""
    logits = O.gemv_f32(routeur, x)
    oi, ow = O.routeur_topk(logits, k)
    sorties, sorties64 = [], []
    for e in oi:
        bl, bi = codeur.synth_expert(graine, 0, int(e), GPT)
        ex = type("E", (), {})()
        ex.attendu = np.concatenate([O.blocs_vers_soa(bl[j], 2880, 2880, bi[j], canonique=True) for j in range(3)])
        s, s64 = _mlp_oracle(ex, x, GPT)
        sorties.append(s)
        sorties64.append(s64)
    ref = O.combiner(avant, np.concatenate(sorties), 2880, ow, k, 2880)
    ref64 = avant.astype(np.float64) + sum(float(ow[i]) * sorties64[i] for i in range(k))
    return oi, ow, ref, ref64


@pytest.mark.parametrize("k", [1, 2, 6, 8])
def test_fused_moe_layer_topk_sizes_and_reused_workspace(fz, k):
    """The bench's encoding (gate and up 2/32, down 1/16) at top-1, 2, 6 and 8. The workspace starts
    as 0xFF bytes and serves two steps in a row, the second adding into the first's residual with
    another x: nothing in the step may depend on the workspace's earlier contents."""
    E = 12
    couche = codeur.CoucheSynthetique(2029, 0, E, GPT, N_delta=(2, 2, 1), N_codes=(32, 32, 16))
    freqs = couche.freqs()
    luts = O.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)])
    parts = [dev(couche.partie(e)) for e in range(E)]
    table = dev(np.array([p.data_ptr() for p in parts], np.uint64))
    rep, ctl0 = zeros(fusion.taille_repertoire(E)), zeros(16)
    fz.monter_couche(vue(table), E, GPT, vue(rep), vue(ctl0))
    assert list(hote(ctl0, np.uint32)) == [0, 0, 0, 0]
    routeur = np.stack([O.synth_normale_bf16(2029, 3, e, 2880, 0.02) for e in range(E)])
    r16 = (routeur.view(np.uint32) >> 16).astype(np.uint16)
    avant = O.synth_normale_bf16(2029, 5, 0, 2880, 1.0)
    l, rd, res = dev(luts), dev(r16), dev(avant)
    tr = dev(np.full(fusion.taille_travail_couche(GPT, E, k, 16), 0xFF, np.uint8))
    for pas in range(2):
        x = O.synth_normale_bf16(2029, 4, pas, 2880, 1.0)
        xd = dev(x)
        idx, w, ctl = zeros(32), zeros(32), zeros(16)
        fz.couche_moe(vue(rep), E, vue(l), GPT, vue(rd), None, vue(xd), k, vue(res), vue(idx), vue(w), vue(ctl),
                      vue(tr), 1, 16)
        got = hote(res, np.float32).copy()
        assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]
        oi, ow, ref, ref64 = _couche_oracle(2029, E, k, x, avant, routeur)
        assert (hote(idx, np.uint32)[:k] == oi).all() and np.abs(hote(w, np.float32)[:k] - ow).max() <= 1e-6
        assert np.abs(got - ref).max() <= TOL * np.abs(ref).max(), (k, pas)
        assert np.abs(got - ref64).max() <= TOL * np.abs(ref64).max(), (k, pas)
        avant = got
    couche.liberer()


@pytest.mark.parametrize("N", [(16, 32), (2, 16)])
def test_fused_moe_router_ties_and_order(fz, N):
    """The fused layer's top-k on tied logits: experts 2 and 9 get identical router rows, as do 5 and
    6, all scaled to win; the selection must be the reference's (logit desc, index asc), i.e. the
    oracle's routeur_topk on the same logits, and the weights its f64 softmax."""
    E, k = 12, 4
    couche = codeur.CoucheSynthetique(2029, 0, E, GPT, N_delta=N[0], N_codes=N[1])
    freqs = couche.freqs()
    luts = O.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)])
    parts = [dev(couche.partie(e)) for e in range(E)]
    table = dev(np.array([p.data_ptr() for p in parts], np.uint64))
    rep, ctl0 = zeros(fusion.taille_repertoire(E)), zeros(16)
    fz.monter_couche(vue(table), E, GPT, vue(rep), vue(ctl0))
    base = np.stack([O.synth_normale_bf16(2029, 3, e, 2880, 0.02) for e in range(E)])
    for t in range(3):
        x = O.synth_normale_bf16(2029, 4, t, 2880, 1.0)
        # rows 2 = 9 and 5 = 6, turned towards x and scaled by 4 (a power of two: still bf16-exact),
        # so that the top-4 is exactly the two tied pairs
        routeur = base.copy()
        for a, b in ((2, 9), (5, 6)):
            r = base[a] * (4.0 if float(base[a] @ x) > 0 else -4.0)
            routeur[a] = routeur[b] = r
        r16 = (routeur.view(np.uint32) >> 16).astype(np.uint16)
        l, rd, xd, res = dev(luts), dev(r16), dev(x), dev(np.zeros(2880, np.float32))
        idx, w, ctl = zeros(32), zeros(32), zeros(16)
        tr = zeros(fusion.taille_travail_couche(GPT, E, k, N[1]))
        fz.couche_moe(vue(rep), E, vue(l), GPT, vue(rd), None, vue(xd), k, vue(res), vue(idx), vue(w), vue(ctl),
                      vue(tr), *N)
        logits = O.gemv_f32(routeur, x)
        oi, ow = O.routeur_topk(logits, k)
        assert sorted(oi) == [2, 5, 6, 9] and logits[2] == logits[9] and logits[5] == logits[6]
        assert (hote(idx, np.uint32)[:k] == oi).all(), (t, hote(idx, np.uint32)[:k], oi)
        assert np.abs(hote(w, np.float32)[:k] - ow).max() <= 1e-6
        assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]
    couche.liberer()


def test_fused_moe_router_nan_never_chosen(fz):
    """A router row of NaN weights gives a NaN logit: the fused layer's top-k must pass over it as the
    reference does (a NaN is never ordered before another logit), and rank the others unchanged:
    rows 2 = 9 tied and scaled to win, row 5 NaN, row 6 scaled to win, so the fourth choice is the
    best of the rest; indices and weights equal the oracle's routeur_topk."""
    E, k, N = 12, 4, (2, 16)
    couche = codeur.CoucheSynthetique(2031, 0, E, GPT, N_delta=N[0], N_codes=N[1])
    freqs = couche.freqs()
    luts = O.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)])
    parts = [dev(couche.partie(e)) for e in range(E)]
    table = dev(np.array([p.data_ptr() for p in parts], np.uint64))
    rep, ctl0 = zeros(fusion.taille_repertoire(E)), zeros(16)
    fz.monter_couche(vue(table), E, GPT, vue(rep), vue(ctl0))
    base = np.stack([O.synth_normale_bf16(2031, 3, e, 2880, 0.02) for e in range(E)])
    for t in range(2):
        x = O.synth_normale_bf16(2031, 4, t, 2880, 1.0)
        routeur = base.copy()
        for a in (2, 6):
            routeur[a] = base[a] * (4.0 if float(base[a] @ x) > 0 else -4.0)
        routeur[9] = routeur[2]
        routeur[5] = np.float32(np.nan)
        r16 = (routeur.view(np.uint32) >> 16).astype(np.uint16)
        l, rd, xd, res = dev(luts), dev(r16), dev(x), dev(np.zeros(2880, np.float32))
        idx, w, ctl = zeros(32), zeros(32), zeros(16)
        tr = zeros(fusion.taille_travail_couche(GPT, E, k, N[1]))
        fz.couche_moe(vue(rep), E, vue(l), GPT, vue(rd), None, vue(xd), k, vue(res), vue(idx), vue(w), vue(ctl),
                      vue(tr), *N)
        logits = O.gemv_f32(routeur, x)
        oi, ow = O.routeur_topk(logits, k)
        assert np.isnan(logits[5]) and 5 not in list(oi) and {2, 6, 9} <= set(int(i) for i in oi)
        assert (hote(idx, np.uint32)[:k] == oi).all(), (t, hote(idx, np.uint32)[:k], oi)
        assert np.abs(hote(w, np.float32)[:k] - ow).max() <= 1e-6
        assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]
    couche.liberer()


@pytest.mark.parametrize("N", [(8, 8), (1, 16)])
def test_fused_moe_layer_bad_parts(fz, N):
    """A layer whose parts all fail the mount checks: the step counts format errors in every pass
    that meets a bad directory entry and leaves the residual alone (nothing is combined)."""
    E, k = 6, 4
    dims = DimsExpert.de([256, 256, 256], [256, 256, 256])
    couche = codeur.CoucheSynthetique(77, 0, E, dims, N_delta=N[0], N_codes=N[1])
    freqs = couche.freqs()
    luts = O.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)])
    mauvaises = []
    for e in range(E):
        p = couche.partie(e).copy()
        p[0] ^= 0xFF  # magic
        mauvaises.append(dev(p))
    table = dev(np.array([p.data_ptr() for p in mauvaises], np.uint64))
    rep, ctl0 = zeros(fusion.taille_repertoire(E)), zeros(16)
    fz.monter_couche(vue(table), E, dims, vue(rep), vue(ctl0))
    assert hote(ctl0, np.uint32)[1] == 3 * E
    r16 = (np.stack([O.synth_normale_bf16(77, 3, e, 256, 0.02) for e in range(E)]).view(np.uint32) >> 16)
    x = O.synth_normale_bf16(77, 4, 0, 256, 1.0)
    residu0 = np.full(256, 0.5, np.float32)
    l, rd, xd, res = dev(luts), dev(r16.astype(np.uint16)), dev(x), dev(residu0)
    idx, w, ctl = zeros(32), zeros(32), zeros(16)
    tr = zeros(fusion.taille_travail_couche(dims, E, k, N[1]))
    fz.couche_moe(vue(rep), E, vue(l), dims, vue(rd), None, vue(xd), k, vue(res), vue(idx), vue(w), vue(ctl),
                  vue(tr), *N)
    c = hote(ctl, np.uint32)
    assert c[1] > 0 and c[0] == 0 and c[2] == 0 and c[3] == 0
    logits = O.gemv_f32(np.stack([O.synth_normale_bf16(77, 3, e, 256, 0.02) for e in range(E)]), x)
    oi, _ = O.routeur_topk(logits, k)
    assert (hote(idx, np.uint32)[:k] == oi).all()
    assert (hote(res, np.float32) == residu0).all()
    couche.liberer()


def test_mount_counts_bad_parts(fz):
    """The layer mount checks every part once: a broken magic and a flipped header byte are format
    errors, the good parts are mounted, and a layer step through a bad entry counts errors again."""
    E, N = 3, (8, 8)
    dims = DimsExpert.de([256, 256, 256], [256, 256, 256])
    couche = codeur.CoucheSynthetique(78, 0, E, dims, N_delta=N[0], N_codes=N[1])
    p0 = couche.partie(0).copy()
    p1 = couche.partie(1).copy()
    p1[0] ^= 0xFF                           # magic
    p2 = couche.partie(2).copy()
    e = 64 + 16 * 3                          # stream descriptor 3 (CODES_CTX of matrix 0): offset not 16-aligned
    p2[e + 4] ^= 0x04
    parts = [dev(p0), dev(p1), dev(p2)]
    table = dev(np.array([p.data_ptr() for p in parts], np.uint64))
    rep, ctl = zeros(fusion.taille_repertoire(E)), zeros(16)
    fz.monter_couche(vue(table), E, dims, vue(rep), vue(ctl))
    c = hote(ctl, np.uint32)
    assert c[0] == 0 and c[2] == 0 and c[1] == 3 + 1   # 3 matrices of part 1, matrix 0 of part 2
    bon = hote(rep, np.uint32).reshape(E * 3, 32)[:, 24]
    assert list(bon) == [1, 1, 1, 0, 0, 0, 0, 1, 1]
    couche.liberer()
