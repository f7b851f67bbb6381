"""Pins the CPU oracle's matrix codec, part format, slot layout and arithmetic (oracle/codec.c,
oracle/maths.c, oracle/synth.c) against the reference's known answers and closed forms.

Reference tests followed: moteur/crates/trc-codec/tests/rans.rs:257-363,
moteur/crates/trc-noyaux/src/abi.rs:340-359, moteur/crates/trc-noyaux/tests/carte.rs:330-554,
moteur/crates/trc-noyaux/tests/passe.rs:203-318, moteur/crates/trc-format/tests/aller_retour.rs:411-416.
"""
import hashlib
import math
import struct

import numpy as np
import pytest

import oracle_ffi as O


def _xs(seed):
    st = [seed]

    def nxt():
        x = st[0]
        x ^= x >> 12
        x ^= (x << 25) & 0xFFFFFFFFFFFFFFFF
        x ^= x >> 27
        st[0] = x
        return (x * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF
    return nxt


def _blocs_mxfp4(rng, r, b):
    """Synthetic MXFP4 rows with scales around a median (shape of tests/rans.rs:258-271)."""
    v = np.zeros((r, b, 17), np.uint8)
    med = 118 + rng.integers(0, 4, r)
    v[:, :, 0] = (med[:, None] + np.minimum(rng.geometric(0.5, (r, b)) - 1, 4) - 2).astype(np.uint8)
    lo = np.minimum(rng.geometric(0.3, (r, b, 16)) - 1, 15)
    hi = np.minimum(rng.geometric(0.3, (r, b, 16)) - 1, 15)
    v[:, :, 1:] = (lo | (hi << 4)).astype(np.uint8)
    return v.reshape(-1)


def _matrice_une(blocs, r, b, freqs, canonique, biais):
    partie, utiles = O.coder_expert([blocs], [biais], [r], [32 * b], [freqs], canonique=canonique)
    return partie, utiles


@pytest.mark.parametrize("r,b", [(64, 2), (90, 3), (2880 // 8, 90)])
def test_matrix_v10_reconstructs_rans_tests_273(r, b):
    rng = np.random.default_rng(r * b)
    blocs = [_blocs_mxfp4(rng, r, b) for _ in range(3)]
    t = O.tables_matrice(blocs, r, b, canonique=False)
    for x in range(3):
        biais = rng.standard_normal(r).astype(np.float32)
        partie, utiles = _matrice_une(blocs[x], r, b, t, False, biais)
        p = O.lire_partie(partie)
        assert p is not None and p.utiles == utiles and p.n_flux == 4
        luts4 = np.concatenate([O.lut(t[i])[1] for i in range(4)])
        codes, ech, bi, bd, bc = O.decoder_matrice(partie, 0, r, b, luts4)
        assert bd.voies_hors_l == 0 and bc.voies_hors_l == 0 and bd.tuiles_mots_faux == 0 and bc.tuiles_mots_faux == 0
        orig = blocs[x].reshape(-1, 17)
        assert (ech == orig[:, 0]).all() and (codes == orig[:, 1:].reshape(-1)).all()
        assert (bi.view(np.uint32) == biais.view(np.uint32)).all()
        # break: a median flipped -> scales wrong
        d = [p.flux[i] for i in range(p.n_flux) if p.flux[i].sorte == 1][0]
        q = bytearray(partie)
        q[d.decalage] ^= 1
        codes2, ech2, *_ = O.decoder_matrice(bytes(q), 0, r, b, luts4)
        assert (ech2 != orig[:, 0]).any()


def test_matrix_v12_canonical_rans_tests_310():
    """Zeros with a random sign: the canonical encoding reconstructs the canonical expert, carries
    no nibble 8, its tables give frequency 0 to the 31 bytes with a nibble 8, and it is cheaper."""
    rng = np.random.default_rng(20261017)
    r, b = 2880 // 8, 90
    blocs = []
    for _ in range(3):
        v = _blocs_mxfp4(rng, r, b).reshape(-1, 17)
        q = v[:, 1:]
        for sh in (0, 4):
            z = ((q >> sh) & 15) == 0
            flip = z & (rng.integers(0, 2, q.shape) == 1)
            q[flip] |= np.uint8(8 << sh)
        blocs.append(v.reshape(-1))
    n8 = sum(int(((x.reshape(-1, 17)[:, 1:] & 15) == 8).sum() + ((x.reshape(-1, 17)[:, 1:] >> 4) == 8).sum()) for x in blocs)
    assert n8 > 0
    porte8 = np.array([(o & 15) == 8 or (o >> 4) == 8 for o in range(256)])
    assert porte8.sum() == 31
    octets = [0, 0]
    for i, canon in enumerate([False, True]):
        t = O.tables_matrice(blocs, r, b, canonique=canon)
        if canon:
            assert (t[1:, porte8] == 0).all()
        luts4 = np.concatenate([O.lut(t[k])[1] for k in range(4)])
        for x in range(3):
            biais = np.zeros(r, np.float32)
            partie, _ = _matrice_une(blocs[x], r, b, t, canon, biais)
            p = O.lire_partie(partie)
            octets[i] += sum(p.flux[k].longueur for k in range(p.n_flux) if p.flux[k].sorte == 4)
            codes, ech, bi, bd, bc = O.decoder_matrice(partie, 0, r, b, luts4)
            assert bd.voies_hors_l == 0 and bc.voies_hors_l == 0
            orig = blocs[x].reshape(-1, 17)[:, 1:].reshape(-1)
            if canon:
                lo, hi = orig & 15, orig >> 4
                lo = np.where(lo == 8, 0, lo)
                hi = np.where(hi == 8, 0, hi)
                attendu = (lo | (hi << 4)).astype(np.uint8)
                assert (codes == attendu).all()
                assert not porte8[codes].any()
                assert (codes != orig).any()
            else:
                assert (codes == orig).all()
    assert (octets[0] - octets[1]) * 8 > 0.5 * n8


def test_median_and_delta_brute_force_tiny():
    """med = sorted(e)[B//2] (ARCHITECTURE.md:653) and delta = (e - med + 128) mod 256, checked on
    every row of tiny matrices with python's own sort."""
    rng = np.random.default_rng(3)
    for R in (1, 5):
        for B in (1, 2, 3):
            bl = rng.integers(0, 256, (R, B, 17)).astype(np.uint8)
            med, delta, qs = O.preparer_matrice(bl.reshape(-1), R, B)
            for r in range(R):
                e = [int(v) for v in bl[r, :, 0]]
                m = sorted(e)[B // 2]
                assert med[r] == m
                for i in range(B):
                    assert delta[r * B + i] == (e[i] - m + 128) % 256
            assert (delta[R * B:] == 0).all() and delta.size % 128 == 0
            assert (qs[:16 * R * B] == bl[:, :, 1:].reshape(-1)).all()


def test_part_reader_refusals():
    rng = np.random.default_rng(9)
    r, b = 64, 2
    bl = _blocs_mxfp4(rng, r, b)
    t = O.tables_matrice([bl], r, b)
    partie, _ = _matrice_une(bl, r, b, t, True, np.zeros(r, np.float32))
    assert len(partie) % 4096 == 0
    assert O.lire_partie(partie) is not None
    for pos, masque, nom in [(0, 0x05, "magic"), (20, 0x05, "reserved header"), (64, 0x40, "unknown kind"),
                             (64 + 3, 0x05, "reserved descriptor"), (64 + 1, 0x07, "matrix index"),
                             (64 + 4, 0x05, "offset alignment")]:
        q = bytearray(partie)
        q[pos] ^= masque
        assert O.lire_partie(bytes(q)) is None, nom
    q = bytearray(partie)
    q[-1] = 1  # non-zero padding
    assert O.lire_partie(bytes(q)) is None


def test_slot_layout_abi_rs_340():
    m = O.disposition_matrice(2880, 2880)
    assert (m.echelles, m.biais, m.pas) == (4_147_200, 4_406_528, 4_418_048)
    assert O.taille_emplacement([2880] * 3, [2880] * 3) == 13_254_144
    assert O.disposition_j([2880] * 3, [2880] * 3, 2).base == 2 * 4_418_048


def test_empreinte64_abc_kat():
    # trc-format/tests/aller_retour.rs:411-416: LE u64 of bytes ba 78 16 bf 8f 01 cf ea
    assert O.empreinte64(b"abc") == 0xEACF018FBF1678BA
    assert O.empreinte64(b"") == struct.unpack("<Q", bytes.fromhex("e3b0c44298fc1c14"))[0]
    rng = np.random.default_rng(0)
    for n in (1, 55, 56, 63, 64, 65, 119, 120, 1000, 4099):
        b = rng.integers(0, 256, n).astype(np.uint8).tobytes()
        assert O.empreinte64(b) == struct.unpack("<Q", hashlib.sha256(b).digest()[:8])[0]


# ------------------------------------------------------------------------------ arithmetic

def test_e8m0_scale_all_256_values():
    for e in range(256):
        assert O.lib().orc_echelle_e8m0(e) == math.ldexp(1.0, e - 128)


def test_e2m1_values_and_code_8_is_zero():
    k = [0, 1, 2, 3, 4, 6, 8, 12]
    for c in range(16):
        v = O.lib().orc_valeur_e2m1x2(c)
        assert abs(v) == k[c & 7] and (c < 8 or v <= 0)
    assert O.lib().orc_valeur_e2m1x2(8) == 0.0


def _expert_exact(seed, r=2880, c=2880):
    """Integer-exact fixture of tests/carte.rs:1-10: scales in [117,123], nibble law 40/40/20 with
    random sign; every GEMV partial sum is exact in f32."""
    rng = np.random.default_rng(seed)
    nb = r * (c // 32)
    e = rng.integers(117, 124, nb).astype(np.uint8)
    u = rng.integers(0, 100, (nb, 32))
    mag = np.where(u < 40, u % 2, np.where(u < 80, 2 + u % 3, 5 + u % 3))
    code = mag | (rng.integers(0, 2, (nb, 32)) << 3)
    qs = (code[:, :16] | (code[:, 16:] << 4)).astype(np.uint8)
    bl = np.zeros((nb, 17), np.uint8)
    bl[:, 0] = e
    bl[:, 1:] = qs
    biais = ((rng.integers(0, 2001, r) - 1000) / 2048.0).astype(np.float32)
    return bl.reshape(-1), biais


def test_gemv_reference_order_exact_on_integer_fixture_carte_rs_330():
    r = c = 2880
    bl, biais = _expert_exact(7)
    mat = O.blocs_vers_soa(bl, r, c, biais, canonique=False)
    x = (np.random.default_rng(11).integers(0, 5, c) - 2).astype(np.float32)
    y = O.gemv_mxfp4(mat, x, r, c)
    y64 = O.gemv_mxfp4_f64(mat, x, r, c)
    assert (y.view(np.uint32) == y64.astype(np.float32).view(np.uint32)).all()
    # break: the reference scaled by 1.01 must be seen
    assert (y != (y64 * 1.01).astype(np.float32)).any()


def test_gemv_reads_code_8_as_0_carte_rs_487():
    r = c = 2880
    bl, biais = _expert_exact(20261017)
    mat = O.blocs_vers_soa(bl, r, c, biais, canonique=False)
    can = O.blocs_vers_soa(bl, r, c, biais, canonique=True)
    assert (mat != can).any()
    rng = np.random.default_rng(17)
    x = (rng.random(c) + 0.5) * np.exp2(rng.integers(-10, 11, c)) * np.where(rng.integers(0, 2, c) == 1, -1, 1)
    x = x.astype(np.float32)
    x[::97] = 0.0
    x[1::97] = -0.0
    assert (O.gemv_mxfp4(mat, x, r, c).view(np.uint32) == O.gemv_mxfp4(can, x, r, c).view(np.uint32)).all()


def test_gemv_f32_router_order_against_f64():
    rng = np.random.default_rng(4)
    W = rng.integers(-8, 8, (128, 2880)).astype(np.float32) / 8
    x = rng.integers(-4, 5, 2880).astype(np.float32) / 4
    y = O.gemv_f32(W, x)
    assert (y == (W.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)).all()  # exact sums


def test_swiglu_fixture_passe_rs_203():
    g = np.array([100.0, 7.0, -3.0, 0.0, 1.5], np.float32)
    u = np.array([100.0, 7.0, -100.0, 5.0, -0.25], np.float32)
    y = O.swiglu_oai(g, u)
    assert y[0].view(np.uint32) == y[1].view(np.uint32)
    for i in range(5):
        gg, uu = min(float(g[i]), 7.0), max(min(float(u[i]), 7.0), -7.0)
        att = gg / (1.0 + math.exp(-1.702 * gg)) * (uu + 1.0)
        assert abs(float(y[i]) - att) <= 1e-6 * max(abs(att), 1e-30)
    assert O.swiglu_oai([0.0], [5.0])[0] == 0.0
    assert O.swiglu_oai([1.0], [-1.0])[0] == 0.0


def test_combiner_bit_equal_to_ordered_f32_sum_passe_rs_304():
    rng = np.random.default_rng(3)
    d = 2880
    x = ((rng.random(d) - 0.5) * 1e3).astype(np.float32)
    s = ((rng.random(4 * d) - 0.5) * 7.0).astype(np.float32)
    w = np.array([0.4123, 0.3001, 0.2, 0.0876], np.float32)
    y = O.combiner(x, s, d, w, 4, d)
    t = w[0] * s[:d]
    for j in range(1, 4):
        t = (t + w[j] * s[j * d:(j + 1) * d]).astype(np.float32)
    assert (y.view(np.uint32) == (x + t).astype(np.float32).view(np.uint32)).all()


def test_router_fixture_passe_rs_275():
    idx, w = O.routeur_topk([1.0, 3.0, 3.0, 0.0, 2.0, -1.0], 4)
    assert list(idx) == [1, 2, 4, 0]
    e = [math.exp(v - 3.0) for v in (3.0, 3.0, 2.0, 1.0)]
    z = sum(e)
    assert [float(v) for v in w] == [float(np.float32(v / z)) for v in e]
    # ties -> lower index (ops.rs:185-191)
    idx, w = O.routeur_topk([1.0, 3.0, 3.0, 0.0, 2.0], 3)
    assert list(idx) == [1, 2, 4] and abs(float(w.sum()) - 1.0) < 1e-6 and w[0] == w[1]


def _topk_biais_par_tri(l, b, k):
    """The reference's host version (tests/passe.rs:328-337): sort by f32 score desc then index,
    keep k, sort those by logit desc then index, f64 softmax of the logits."""
    l = np.asarray(l, np.float32)
    sc = (l + np.asarray(b, np.float32)).astype(np.float32)
    ids = sorted(range(l.size), key=lambda i: (-float(sc[i]), i))[:k]
    ids = sorted(ids, key=lambda i: (-float(l[i]), i))
    m = float(l[ids[0]])
    e = [math.exp(float(l[i]) - m) for i in ids]
    z = 0.0
    for v in e:
        z += v
    return ids, [float(np.float32(v / z)) for v in e]


def test_biased_router_hand_case_and_zero_bias():
    # scores [1, 3, 3, 5, 2, -1]: chosen {3, 1, 2, 4}, returned by logit: 1, 2 (3.0), 4 (2.0), 3 (0.0)
    l = [1.0, 3.0, 3.0, 0.0, 2.0, -1.0]
    idx, w = O.routeur_topk_biais(l, [0, 0, 0, 5.0, 0, 0], 4)
    assert list(idx) == [1, 2, 4, 3]
    e = [1.0, 1.0, math.exp(-1.0), math.exp(-3.0)]
    z = ((e[0] + e[1]) + e[2]) + e[3]
    assert [float(v) for v in w] == [float(np.float32(v / z)) for v in e]
    # zero bias: routeur_topk bit for bit
    rng = np.random.default_rng(7)
    for E in (6, 32, 256):
        lg = (rng.integers(-40, 41, E) * 0.25).astype(np.float32)
        i0, w0 = O.routeur_topk(lg, 4)
        i1, w1 = O.routeur_topk_biais(lg, np.zeros(E, np.float32), 4)
        assert (i0 == i1).all() and (w0.view(np.uint32) == w1.view(np.uint32)).all()


def test_biased_router_equals_sort_based_restatement():
    """Tie-forcing draws as tests/passe.rs:339-393: logits on a 0.25 grid, E in {6, 32, 256},
    beta in {0, 0.041, 0.3, 1}, random masks; the bias changes some sets."""
    rng = np.random.default_rng(20261027)
    changes = 0
    for essai in range(160):
        E = [6, 32, 32, 256][essai % 4]
        beta = [0.0, 0.041, 0.3, 1.0][(essai // 4) % 4]
        l = (rng.integers(-40, 41, E) * 0.25).astype(np.float32)
        b = np.where(rng.integers(0, 2, E) == 1, beta, 0.0).astype(np.float32)
        idx, w = O.routeur_topk_biais(l, b, 4)
        ri, rw = _topk_biais_par_tri(l, b, 4)
        assert list(idx) == ri, essai
        assert [float(v) for v in w] == rw, essai
        if sorted(ri) != sorted(_topk_biais_par_tri(l, np.zeros(E), 4)[0]):
            changes += 1
    assert changes > 5


# ------------------------------------------------------------------------------ generators

def test_splitmix64_kat():
    # Vigna's splitmix64 from state 0
    assert O.splitmix64_suite(0, 3) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_xorshift64s_closed_form():
    nxt = _xs(1)
    assert O.xorshift_suite(1, 5) == [nxt() for _ in range(5)]


def test_synthetic_workload_statistics():
    bl, bi = O.synth_matrice(2026, 0, 3, 2, 2880, 2880)
    b = bl.reshape(-1, 17)
    assert b[:, 0].min() == 119 and b[:, 0].max() == 125
    nib = np.concatenate([b[:, 1:] & 15, b[:, 1:] >> 4], axis=None)
    p = np.bincount(nib, minlength=16) / nib.size
    attendu = [0.10, 0.14, 0.13, 0.06, 0.035, 0.02, 0.01, 0.005] * 2
    assert np.abs(p - attendu).max() < 0.002
    assert abs(float(bi.std()) - 0.02) < 0.002
    assert (bi == bi.astype(np.float32)).all()
    bits = bi.view(np.uint32)
    assert (bits & 0xFFFF == 0).all()  # bf16-valued
    bl2, _ = O.synth_matrice(2026, 0, 3, 2, 2880, 2880)
    assert (bl2 == bl).all()
    bl3, _ = O.synth_matrice(2026, 0, 4, 2, 2880, 2880)
    assert (bl3 != bl).any()
