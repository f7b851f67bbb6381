"""GPU parity of the reference kernel API (decoder, raw copy, GEMV, router, SwiGLU, combine) against
the CPU oracle, through the C-ABI. Witnesses follow moteur/crates/trc-noyaux/tests/carte.rs and
tests/passe.rs: exact slot bytes and zero control words, breaks that must be seen, batch == single,
bit-exact GEMV on integer-exact data and on the synthetic workload, code 8 read as 0."""
import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle_ffi as O  # noqa: E402
from gpu_outils import DEV, Expert, dev, hote, vue, zeros  # noqa: E402
from troncons_amd import codeur  # noqa: E402
from troncons_amd import noyaux as K  # noqa: E402
from troncons_amd.noyaux import DescDecodage, DescGemv, DimsExpert, VueCarte  # noqa: E402

GPT = DimsExpert.gpt_oss()
TE = 13_254_144


@pytest.fixture(scope="module")
def k():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return K.Noyaux()


def _decoder(k, partie: bytes, luts, brut=False, grilles=None, dims=GPT):
    te = K.taille_emplacement(dims)
    p = dev(partie)
    l = dev(luts)
    e = zeros(te)
    ctl = zeros(16)
    if brut:
        k.copier_brut(vue(p), vue(e), dims, vue(ctl))
    elif grilles is not None:
        k.decoder_expert_grilles(vue(p), vue(e), vue(l), dims, vue(ctl), grilles)
    else:
        k.decoder_expert(vue(p), vue(e), vue(l), dims, vue(ctl))
    return hote(e), hote(ctl, np.uint32)


@pytest.fixture(scope="module")
def expert_ref():
    return Expert(2026_10_15, GPT)


@pytest.mark.parametrize("N", [(256, 256), (32, 32), (8, 16)])
def test_decoder_exact_against_oracle(k, N):
    ex = Expert(2026_10_15 + N[1], GPT, N_delta=N[0], N_codes=N[1])
    empl, ctl = _decoder(k, ex.partie, ex.luts)
    assert list(ctl) == [0, 0, 0, 0]
    assert (empl == ex.attendu).all()
    oracle, octl = O.decoder_expert(ex.partie, ex.luts, [2880] * 3, [2880] * 3)
    assert list(octl) == [0, 0, 0, 0] and (oracle == empl).all()
    # grids read from the part give the same bytes
    g = K.grilles_depuis_partie(ex.partie)
    empl2, ctl2 = _decoder(k, ex.partie, ex.luts, grilles=g)
    assert list(ctl2) == [0, 0, 0, 0] and (empl2 == empl).all()


# Blocks per row 1, 1, 2 (8200 rows: more than the 8192 medians kept in LDS), then 3, 3, 5.
RAGGED = [DimsExpert.de([37, 37, 8200], [32, 32, 64]), DimsExpert.de([5, 5, 70], [96, 96, 160])]


@pytest.mark.parametrize("forme", [0, 1])
@pytest.mark.parametrize("N", [(3, 7), (5, 16), (256, 256), (2, 33)])
def test_decoder_ragged_shapes_against_oracle(k, N, forme):
    """Rows of 1-3 blocks (a lane's 4 deltas and a context group's blocks span several rows), a matrix
    whose medians are read from device memory, tile lengths that are not multiples of the 16
    macro-steps a CODES context group covers, stream padding past the last block; the raw copy of
    the same matrices (region lengths that are not multiples of 16 bytes)."""
    print(f"ragged decoder N {N} shape {forme}", flush=True)
    dims = RAGGED[forme]
    ex = Expert(2027 + N[0] * 100 + N[1] + forme, dims, N_delta=N[0], N_codes=N[1])
    empl, ctl = _decoder(k, ex.partie, ex.luts, dims=dims)
    assert list(ctl) == [0, 0, 0, 0]
    oracle, octl = O.decoder_expert(ex.partie, ex.luts, dims.lignes, dims.colonnes)
    assert list(octl) == [0, 0, 0, 0] and (oracle == empl).all()
    assert (empl == ex.attendu).all()
    p_brut, attendu_brut = ex.partie_brute()
    sentinelle = zeros(K.taille_emplacement(dims))
    sentinelle.fill_(0xA5)
    ctl = zeros(16)
    k.copier_brut(vue(dev(p_brut)), vue(sentinelle), dims, vue(ctl))
    got = hote(sentinelle)
    assert hote(ctl, np.uint32)[1] == 0
    for j in range(3):  # region bytes equal, the slot's alignment padding untouched
        d = K.disposition(dims, j)
        R, C_ = dims.lignes[j], dims.colonnes[j]
        nb = R * (C_ // 32)
        for deb, lon in ((0, 16 * nb), (d.echelles, nb), (d.biais, 4 * R)):
            a = d.base + deb
            assert (got[a:a + lon] == attendu_brut[a:a + lon]).all(), (j, deb)
        assert (got[d.base + 16 * nb:d.base + d.echelles] == 0xA5).all()
        assert (got[d.base + d.echelles + nb:d.base + d.biais] == 0xA5).all()


def test_gemv_ragged_shapes_bit_exact(k):
    """The reference-order GEMVs on rows of 1-3 blocks and row counts that fill neither a half's row
    pair nor a block's 16 rows; gemv_f32 on 37 rows of 37 quads (a lane's batch of four never
    whole), with and without bias."""
    rng = np.random.default_rng(3)
    for f, dims in enumerate(RAGGED):
        ex = Expert(2028 + f, dims, N_delta=16, N_codes=16)
        empl = dev(ex.attendu)
        for j in range(3):
            R, C_ = dims.lignes[j], dims.colonnes[j]
            d = K.disposition(dims, j)
            x = O.synth_normale_bf16(5, j, f, C_, 1.0)
            y = zeros(4 * R)
            k.gemv(vue(empl, d.base, d.pas), vue(dev(x)), vue(y), R, C_)
            ref = O.gemv_mxfp4(ex.attendu[d.base:d.base + d.pas], x, R, C_)
            assert (hote(y, np.uint32) == ref.view(np.uint32)).all(), (f, j)
    for R, C_ in ((37, 148), (1, 4), (33, 4 * 129)):
        W = rng.standard_normal((R, C_)).astype(np.float32)
        x = rng.standard_normal(C_).astype(np.float32)
        b = rng.standard_normal(R).astype(np.float32)
        y = zeros(4 * R)
        k.gemv_f32(vue(dev(W)), vue(dev(x)), vue(dev(b)), vue(y), R, C_)
        assert (hote(y, np.uint32) == O.gemv_f32(W, x, b).view(np.uint32)).all(), (R, C_)
        k.gemv_f32(vue(dev(W)), vue(dev(x)), None, vue(y), R, C_)
        assert (hote(y, np.uint32) == O.gemv_f32(W, x).view(np.uint32)).all(), (R, C_)


def test_decoder_breaks_are_seen_carte_rs_247(k, expert_ref):
    ex = expert_ref
    p_brut, attendu_brut = ex.partie_brute()
    empl, ctl = _decoder(k, p_brut, ex.luts, brut=True)
    assert ctl[1] == 0 and (empl == attendu_brut).all()
    # 1. one slot of a CODES_CTX LUT (kappa = 1, matrix 0) corrupted
    luts = ex.luts.copy()
    luts[4096 + 4096 // 2] ^= 1
    empl, _ = _decoder(k, ex.partie, luts)
    assert (empl != ex.attendu).any()
    # 2. a bit flipped in the middle of CODES_CTX of matrix 1 (stream 7)
    p = bytearray(ex.partie)
    e = 64 + 16 * 7
    dec = int.from_bytes(p[e + 4:e + 8], "little")
    lon = int.from_bytes(p[e + 8:e + 12], "little")
    p[dec + lon // 2] ^= 0x10
    empl, ctl = _decoder(k, bytes(p), ex.luts)
    assert ctl[0] > 0 and (empl != ex.attendu).any()
    # 3. a part without its magic: format error, nothing decoded
    p = bytearray(ex.partie)
    p[0] ^= 0xFF
    _, ctl = _decoder(k, bytes(p), ex.luts)
    assert ctl[1] > 0


def test_decoder_batch_equals_single_carte_rs_283(k):
    exs = [Expert(100 + i, GPT, N_delta=64, N_codes=64) for i in range(3)]
    parties = [bytearray(e.partie) for e in exs]
    e7 = 64 + 16 * 7
    dec = int.from_bytes(parties[1][e7 + 4:e7 + 8], "little")
    lon = int.from_bytes(parties[1][e7 + 8:e7 + 12], "little")
    parties[1][dec + lon // 2] ^= 0x10
    p = [dev(bytes(x)) for x in parties]
    l = [dev(e.luts) for e in exs]
    empl = zeros(3 * TE)
    ctl = zeros(48)
    descs = b"".join(DescDecodage(p[i].data_ptr(), empl.data_ptr() + i * TE, l[i].data_ptr(),
                                  ctl.data_ptr() + 16 * i).octets() for i in range(3))
    dd = dev(descs)
    k.decoder_lot(vue(dd), 3, GPT)
    tout = hote(empl)
    c = hote(ctl, np.uint32).reshape(3, 4)
    for i in (0, 2):
        assert list(c[i]) == [0, 0, 0, 0]
        assert (tout[i * TE:(i + 1) * TE] == exs[i].attendu).all()
    assert c[1][0] > 0
    seul1, c1 = _decoder(k, bytes(parties[1]), exs[1].luts)
    assert (seul1 == tout[TE:2 * TE]).all() and list(c1) == list(c[1])


def _expert_exact(seed, r=2880, c=2880):
    rng = np.random.default_rng(seed)
    nb = r * (c // 32)
    e = rng.integers(117, 124, nb).astype(np.uint8)
    u = rng.integers(0, 100, (nb, 32))
    mag = np.where(u < 40, u % 2, np.where(u < 80, 2 + u % 3, 5 + u % 3))
    code = mag | (rng.integers(0, 2, (nb, 32)) << 3)
    bl = np.zeros((nb, 17), np.uint8)
    bl[:, 0] = e
    bl[:, 1:] = (code[:, :16] | (code[:, 16:] << 4)).astype(np.uint8)
    biais = ((rng.integers(0, 2001, r) - 1000) / 2048.0).astype(np.float32)
    return bl.reshape(-1), biais


def test_gemv_bit_exact_and_batch_equals_single_carte_rs_330(k):
    r = c = 2880
    mats = []
    for j in range(3):
        bl, bi = _expert_exact(7 + j)
        mats.append(O.blocs_vers_soa(bl, r, c, bi, canonique=False))
    pas = mats[0].size
    empl = dev(np.concatenate(mats))
    xs = np.random.default_rng(11).choice(np.array([-2.0, -1.0, 1.0, 2.0], np.float32), 3 * c)
    x = dev(xs)
    y = zeros(12 * r)
    yl = zeros(12 * r)
    descs = b""
    for j in range(3):
        m = vue(empl, j * pas, pas)
        k.gemv(m, vue(x, 4 * c * j, 4 * c), vue(y, 4 * r * j, 4 * r), r, c)
        descs += bytes(DescGemv(m.adresse, x.data_ptr() + 4 * c * j, yl.data_ptr() + 4 * r * j, r, c))
    dd = dev(descs)
    k.gemv_lot(vue(dd), 3, r)
    ys = hote(y, np.float32)
    assert (ys.view(np.uint32) == hote(yl, np.uint32)).all()
    for j in range(3):
        ref = O.gemv_mxfp4_f64(mats[j], xs[j * c:(j + 1) * c], r, c).astype(np.float32)
        assert (ys[j * r:(j + 1) * r].view(np.uint32) == ref.view(np.uint32)).all()


def test_gemv_bit_exact_on_the_synthetic_workload(k, expert_ref):
    """Same operation order as the reference (gemv.cuh:60-126): every bit equals the oracle's
    restatement of that order, on the BASELINE distribution with full-mantissa x."""
    r = c = 2880
    x = O.synth_normale_bf16(1, 2, 3, c, 1.0)
    empl = dev(expert_ref.attendu)
    xd = dev(x)
    y = zeros(4 * r)
    pas = K.disposition_matrice(r, c).pas
    for j in range(3):
        k.gemv(vue(empl, j * pas, pas), vue(xd), vue(y), r, c)
        got = hote(y, np.float32)
        ref = O.gemv_mxfp4(expert_ref.attendu[j * pas:(j + 1) * pas], x, r, c)
        assert (got.view(np.uint32) == ref.view(np.uint32)).all()
        ref64 = O.gemv_mxfp4_f64(expert_ref.attendu[j * pas:(j + 1) * pas], x, r, c)
        assert np.abs(got - ref64).max() <= 1e-5 * np.abs(ref64).max()


def test_gemv_reads_code_8_as_0_carte_rs_487(k):
    r = c = 2880
    bl, bi = _expert_exact(20261017)
    orig = O.blocs_vers_soa(bl, r, c, bi, canonique=False)
    can = O.blocs_vers_soa(bl, r, c, bi, canonique=True)
    rng = np.random.default_rng(17)
    x = ((rng.random(c) + 0.5) * np.exp2(rng.integers(-10, 11, c)) * np.where(rng.integers(0, 2, c) == 1, -1, 1)).astype(np.float32)
    x[::97] = 0.0
    x[1::97] = -0.0
    xd = dev(x)

    def g(m):
        md, y = dev(m), zeros(4 * r)
        k.gemv(vue(md), vue(xd), vue(y), r, c)
        return hote(y, np.uint32)
    a, b = g(orig), g(can)
    assert (a == b).all()
    casse = can.copy()
    i = next(i for i in range(32) if ((casse[i % 16] >> (4 if i >= 16 else 0)) & 15) == 0 and x[i] != 0)
    casse[i % 16] |= 0x10 if i >= 16 else 0x01
    assert g(casse)[0] != b[0]


def test_gemv_f32_router_bit_exact(k):
    rng = np.random.default_rng(5)
    W = np.stack([O.synth_normale_bf16(7, 3, e, 2880, 0.02) for e in range(128)])
    x = O.synth_normale_bf16(7, 4, 0, 2880, 1.0)
    b = rng.standard_normal(128).astype(np.float32)
    y = zeros(512)
    k.gemv_f32(vue(dev(W)), vue(dev(x)), vue(dev(b)), vue(y), 128, 2880)
    assert (hote(y, np.uint32) == O.gemv_f32(W, x, b).view(np.uint32)).all()
    k.gemv_f32(vue(dev(W)), vue(dev(x)), None, vue(y), 128, 2880)
    assert (hote(y, np.uint32) == O.gemv_f32(W, x).view(np.uint32)).all()


def test_swiglu_router_mailbox_combiner_passe_rs(k):
    g = np.array([100.0, 7.0, -3.0, 0.0, 1.5], np.float32)
    u = np.array([100.0, 7.0, -100.0, 5.0, -0.25], np.float32)
    yv = zeros(20)
    k.swiglu_oai(vue(dev(g)), vue(dev(u)), vue(yv), 5)
    yy = hote(yv, np.float32)
    assert yy[0].view(np.uint32) == yy[1].view(np.uint32)
    for i in range(5):
        gg, uu = min(float(g[i]), 7.0), max(min(float(u[i]), 7.0), -7.0)
        att = gg / (1.0 + math.exp(-1.702 * gg)) * (uu + 1.0)
        assert abs(float(yy[i]) - att) <= 1e-6 * max(abs(att), 1e-30)
    big_g = O.synth_normale_bf16(2, 9, 1, 5760, 3.0)
    big_u = O.synth_normale_bf16(2, 9, 2, 5760, 3.0)
    yv = zeros(4 * 5760)
    k.swiglu_oai(vue(dev(big_g)), vue(dev(big_u)), vue(yv), 5760)
    ref = O.swiglu_oai(big_g, big_u)
    got = hote(yv, np.float32)
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()

    # router: ties broken by the lower index; mapped mailbox protocol
    l = np.array([1.0, 3.0, 3.0, 0.0, 2.0, -1.0], np.float32)
    iv, pv = zeros(16), zeros(16)
    boite = torch.zeros(1024, dtype=torch.int32).pin_memory()
    k.routeur_topk(vue(dev(l)), 6, 4, vue(iv), vue(pv), boite.data_ptr(), 77)
    idx = hote(iv, np.uint32)
    assert list(idx) == [1, 2, 4, 0]
    e = [math.exp(v - 3.0) for v in (3.0, 3.0, 2.0, 1.0)]
    z = sum(e)
    pw = hote(pv, np.float32)
    assert [float(w) for w in pw] == [float(np.float32(v / z)) for v in e]
    mots = boite.numpy()[:9].view(np.uint32)
    assert mots[0] == 77 and list(mots[1:5]) == list(idx) and (mots[5:9].view(np.float32) == pw).all()
    lg = np.random.default_rng(1).standard_normal(128).astype(np.float32)
    k.routeur_topk(vue(dev(lg)), 128, 4, vue(iv), vue(pv))
    oi, ow = O.routeur_topk(lg, 4)
    assert (hote(iv, np.uint32) == oi).all() and np.abs(hote(pv, np.float32) - ow).max() <= 1e-6

    # combine: bit-equal to the ordered f32 host sum
    rng = np.random.default_rng(3)
    d = 2880
    x = ((rng.random(d) - 0.5) * 1e3).astype(np.float32)
    s = ((rng.random(4 * d) - 0.5) * 7.0).astype(np.float32)
    w = np.array([0.4123, 0.3001, 0.2, 0.0876], np.float32)
    xv = dev(x)
    k.combiner(vue(xv), vue(dev(s)), d, vue(dev(w)), 4, d)
    assert (hote(xv, np.uint32) == O.combiner(x, s, d, w, 4, d).view(np.uint32)).all()


def test_biased_router_equals_oracle_and_plain_router_without_bias():
    """tests/passe.rs:320-393: routeur_topk_biais equals the oracle bit for bit (indices and
    weights) on tie-forcing draws (logits on a 0.25 grid, E in {6, 32, 256}, beta in {0, 0.041,
    0.3, 1}, random masks); with a zero bias it equals routeur_topk; the inverted mask gives a
    different answer several times (the test bites) and the bias changes several sets."""
    k = K.Noyaux()
    rng = np.random.default_rng(20261027)
    changes = inverses = 0
    iv, pv, jv, qv = zeros(32), zeros(32), zeros(32), zeros(32)
    for essai in range(160):
        E = [6, 32, 32, 256][essai % 4]
        beta = [0.0, 0.041, 0.3, 1.0][(essai // 4) % 4]
        l = (rng.integers(-40, 41, E) * 0.25).astype(np.float32)
        m = rng.integers(0, 2, E) == 1
        b = np.where(m, beta, 0.0).astype(np.float32)
        bi = np.where(m, 0.0, beta).astype(np.float32)
        lv = dev(l)
        k.routeur_topk_biais(vue(lv), vue(dev(b)), E, 4, vue(iv), vue(pv))
        oi, ow = O.routeur_topk_biais(l, b, 4)
        assert (hote(iv, np.uint32)[:4] == oi).all(), essai
        assert (hote(pv, np.uint32)[:4] == ow.view(np.uint32)).all(), essai
        k.routeur_topk_biais(vue(lv), vue(dev(np.zeros(E, np.float32))), E, 4, vue(iv), vue(pv))
        k.routeur_topk(vue(lv), E, 4, vue(jv), vue(qv))
        assert (hote(iv, np.uint32)[:4] == hote(jv, np.uint32)[:4]).all(), essai
        assert (hote(pv, np.uint32)[:4] == hote(qv, np.uint32)[:4]).all(), essai
        if beta > 0:
            if sorted(O.routeur_topk(l, 4)[0]) != sorted(oi):
                changes += 1
            k.routeur_topk_biais(vue(lv), vue(dev(bi)), E, 4, vue(iv), vue(pv))
            if (hote(iv, np.uint32)[:4] != oi).any():
                inverses += 1
    assert changes > 5 and inverses > 5
    # mailbox: the same words as routeur_topk's
    l = np.array([1.0, 3.0, 3.0, 0.0, 2.0, -1.0], np.float32)
    boite = torch.zeros(1024, dtype=torch.int32).pin_memory()
    k.routeur_topk_biais(vue(dev(l)), vue(dev(np.array([0, 0, 0, 5, 0, 0], np.float32))), 6, 4, vue(iv), vue(pv),
                         boite.data_ptr(), 91)
    torch.cuda.synchronize()
    mots = boite.numpy()[:9].view(np.uint32)
    assert mots[0] == 91 and list(mots[1:5]) == [1, 2, 4, 3]
    assert (mots[5:9] == hote(pv, np.uint32)[:4]).all()
