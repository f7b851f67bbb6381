"""The oracle's forward-pass operations (oracle/passe.c) pinned on the CPU: the reference's own
fixtures (moteur/crates/trc-noyaux/tests/passe.rs, trc-reference/src/ops.rs tests), closed forms,
and numpy where it computes the same thing (f16 rounding, f64 sums)."""
import math

import numpy as np
import pytest

import oracle_ffi as O


class Alea:
    """splitmix64 as tests/passe.rs:58-71 (state advanced first)."""

    def __init__(self, graine):
        self.e = graine

    def suivant(self):
        self.e = (self.e + 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        z = self.e
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & 0xFFFFFFFFFFFFFFFF
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & 0xFFFFFFFFFFFFFFFF
        return z ^ (z >> 31)

    def entre(self, a, b):
        return a + self.suivant() % (b - a + 1)


def f16_puissance(e):
    return (e + 15) << 10


def q8_0_entier(a, r, c):
    """The integer-exact Q8_0 fixture of tests/passe.rs:86-105: d = 2^e, e in [-2, 1], q in
    [-127, 127], x in {-1, 0, 1}, integer bias; the f64 sum is exact in f32."""
    nb = c // 32
    o = np.zeros(r * nb * 34, np.uint8)
    attendu = np.zeros(r)
    x = np.array([a.entre(-1, 1) for _ in range(c)], np.float32)
    biais = np.array([a.entre(-9, 9) for _ in range(r)], np.float32)
    for i in range(r):
        for j in range(nb):
            e = a.entre(-2, 1)
            k = (i * nb + j) * 34
            o[k:k + 2] = np.frombuffer(np.uint16(f16_puissance(e)).tobytes(), np.uint8)
            q = np.array([a.entre(-127, 127) for _ in range(32)], np.int64)
            o[k + 2:k + 34] = q.astype(np.int8).view(np.uint8)
            attendu[i] += 2.0 ** e * float(q @ x[j * 32:(j + 1) * 32].astype(np.int64))
        attendu[i] += biais[i]
    return o, x, biais, attendu


def test_f16_known_answers():
    # tests/passe.rs:154-159: exact values, then ties to even
    k = np.array([1.0, -2.5, 0.0, 65504.0, 1.0 + 2.0 ** -11, 1.0 + 3.0 * 2.0 ** -11, -0.0, 6.1035156e-5], np.float32)
    assert list(O.f16_depuis_f32(k)) == [0x3C00, 0xC100, 0x0000, 0x7BFF, 0x3C00, 0x3C02, 0x8000, 0x0400]


def test_f16_against_numpy():
    # every f16 widens exactly; random f32 in every regime round like numpy's float16 (RNE)
    h = np.arange(65536, dtype=np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = O.f32_depuis_f16(h)
    nan = np.isnan(ref)
    assert (np.isnan(got) == nan).all() and (got[~nan].view(np.uint32) == ref[~nan].view(np.uint32)).all()
    rng = np.random.default_rng(5)
    v = np.concatenate([rng.standard_normal(4000).astype(np.float32),
                        (rng.standard_normal(4000) * 2.0 ** rng.integers(-30, -10, 4000)).astype(np.float32),
                        rng.uniform(60000, 70000, 2000).astype(np.float32),
                        (h[:4096].view(np.float16).astype(np.float32) * np.float32(1 + 2 ** -11)),
                        np.array([np.inf, -np.inf, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26, 65520.0, 65519.99],
                                 np.float32)])
    v = v[np.isfinite(v) | np.isinf(v)]
    with np.errstate(over="ignore"):
        attendu = v.astype(np.float16).view(np.uint16)
    assert (O.f16_depuis_f32(v) == attendu).all()


@pytest.mark.parametrize("r,c", [(37, 96), (300, 1024)])
def test_gemv_q8_0_integer_exact(r, c):
    a = Alea(31)
    o, x, biais, attendu = q8_0_entier(a, r, c)
    y = O.gemv_q8_0(o, x, biais, r, c)
    assert (y == attendu.astype(np.float32)).all()
    # a transposed or shifted operand breaks it
    assert not (O.gemv_q8_0(o, np.roll(x, 1), biais, r, c) == attendu.astype(np.float32)).all()


def test_gemv_q8_0_random_against_f64():
    rng = np.random.default_rng(3)
    r, c = 64, 2880
    nb = c // 32
    d = rng.standard_normal(r * nb).astype(np.float16)
    q = rng.integers(-128, 128, size=(r * nb, 32)).astype(np.int8)
    blocs = np.concatenate([d.view(np.uint8).reshape(-1, 2), q.view(np.uint8)], axis=1).ravel()
    x = rng.standard_normal(c).astype(np.float32)
    W = (d.astype(np.float64)[:, None] * q.astype(np.float64)).reshape(r, c)
    ref = W @ x.astype(np.float64)
    y = O.gemv_q8_0(blocs, x, None, r, c)
    assert np.abs(y - ref).max() <= 1e-6 * np.abs(ref).max()


def test_ligne_q8_0_exact():
    # tests/passe.rs:128-145
    a = Alea(7)
    lignes, c = 5, 64
    o = np.zeros(lignes * 2 * 34, np.uint8)
    for b in range(lignes * 2):
        o[b * 34:b * 34 + 2] = np.frombuffer(np.uint16(f16_puissance(a.entre(-14, 15))).tobytes(), np.uint8)
        o[b * 34 + 2:b * 34 + 34] = np.array([a.entre(-128, 127) for _ in range(32)], np.int64).astype(np.int8).view(np.uint8)
    for l in range(lignes):
        y = O.ligne_q8_0(o, l, c)
        for i in range(c):
            blk = o[(l * 2 + i // 32) * 34:]
            e = (int(blk[0]) | int(blk[1]) << 8) >> 10
            assert y[i] == np.float32(2.0 ** (e - 15) * int(np.int8(blk[2 + i % 32]))), (l, i)


def test_rmsnorm_against_f64():
    # tests/passe.rs:166-176
    a = Alea(11)
    n = 2880
    x = np.array([a.entre(-1000, 1000) / 37.0 for _ in range(2 * n)], np.float32)
    w = np.array([a.entre(1, 300) / 100.0 for _ in range(n)], np.float32)
    y = O.rmsnorm(x, w, n, 2, 1e-5)
    for l in range(2):
        xs = x[l * n:(l + 1) * n].astype(np.float64)
        r = 1.0 / math.sqrt(float((xs * xs).sum()) / n + float(np.float32(1e-5)))
        att = xs * r * w.astype(np.float64)
        assert np.abs(y[l * n:(l + 1) * n] - att).max() <= 1e-6 * np.abs(att).max()
    # eps matters: a zero row gives zeros, not NaN
    assert (O.rmsnorm(np.zeros(256, np.float32), np.ones(256, np.float32), 256, 1, 1e-5) == 0).all()


def test_yarn_ramp_bounds_and_variants():
    # trc-reference ops.rs:146-163
    p = O.rope_gpt_oss()
    l = O.rope_gpt_oss(variante=1)
    _, m, bas, haut = O.inv_freq_yarn(p, 0)
    assert abs(bas - 8.0928) < 1e-3 and abs(haut - 17.3981) < 1e-3
    _, _, lb, lh = O.inv_freq_yarn(l, 0)
    assert (lb, lh) == (8.0, 18.0)
    assert abs(m - (0.1 * math.log(32.0) + 1.0)) < 1e-15
    for i in list(range(8)) + list(range(18, 32)):
        assert O.inv_freq_yarn(p, i)[0] == O.inv_freq_yarn(l, i)[0], i
    assert O.inv_freq_yarn(p, 12)[0] != O.inv_freq_yarn(l, 12)[0]
    # outside the ramp: extrapolation below, interpolation (/32) above
    assert O.inv_freq_yarn(p, 2)[0] == 1.0 / 150000.0 ** (4 / 64)
    assert abs(O.inv_freq_yarn(p, 30)[0] - 1.0 / (32.0 * 150000.0 ** (60 / 64))) < 1e-18


def test_rope_closed_forms():
    a = Alea(11)
    q = np.array([a.entre(-500, 500) / 64.0 for _ in range(64 * 64)], np.float32)
    k = np.array([a.entre(-500, 500) / 64.0 for _ in range(8 * 64)], np.float32)
    p = O.rope_gpt_oss()
    m = 0.1 * math.log(32.0) + 1.0
    # position 0: cos 1, sin 0, every element times the concentration (tests/passe.rs:177-185)
    q0, k0 = O.rope_yarn(q, k, 64, 8, 0, p)
    assert np.abs(q0 - q.astype(np.float64) * m).max() <= 1e-6 * np.abs(q * m).max()
    # factor 1 at position 1000: plain RoPE, inv_freq_i = theta^(-2i/d) (tests/passe.rs:186-200)
    _, k1 = O.rope_yarn(q[:64], k, 1, 8, 1000, O.rope_gpt_oss(facteur=1.0))
    att = np.zeros(8 * 64)
    for h in range(8):
        for i in range(32):
            ang = 1000.0 * 150000.0 ** (-(2 * i) / 64.0)
            s, c = math.sin(ang), math.cos(ang)
            x1, x2 = float(k[h * 64 + i]), float(k[h * 64 + i + 32])
            att[h * 64 + i] = x1 * c - x2 * s
            att[h * 64 + i + 32] = x2 * c + x1 * s
    assert np.abs(k1 - att).max() <= 1e-6 * np.abs(att).max()
    # the norm is kept up to concentration^2 (ops.rs:165-173)
    x = np.sin(np.arange(64) * 0.37).astype(np.float32)
    xr, _ = O.rope_yarn(x, np.zeros(64, np.float32), 1, 0, 333, p)
    n0 = float((x.astype(np.float64) ** 2).sum())
    assert abs(float((xr.astype(np.float64) ** 2).sum()) / n0 - m * m) < 1e-6


def test_ecrire_kv_slot():
    k = np.array([1.0, -2.5, 0.0, 65504.0, 1.0 + 2.0 ** -11, 1.0 + 3.0 * 2.0 ** -11, -0.0, 6.1035156e-5], np.float32)
    ck, cv = O.ecrire_kv(k, -k, np.zeros(8 * 3, np.uint16), np.zeros(8 * 3, np.uint16), 8, 2)
    assert list(ck[16:]) == [0x3C00, 0xC100, 0x0000, 0x7BFF, 0x3C00, 0x3C02, 0x8000, 0x0400]
    assert (ck[:16] == 0).all() and (cv[16:] == (ck[16:] ^ 0x8000)).all()


UN16 = 0x3C00


def f16_entier(n):
    return int(np.float16(n).view(np.uint16))


def test_attention_sink_and_ring():
    dkv = 8 * 64
    # one key, q = 0, sink 0: weight 1/2 (ops.rs:175-186, tests/passe.rs:222-245)
    ck = np.full(dkv, UN16, np.uint16)
    cv = np.array([f16_entier(t % 64) for t in range(dkv)], np.uint16)
    o = O.attention(np.zeros(64 * 64, np.float32), ck, cv, np.zeros(64, np.float32), O.attention_gpt_oss(0, 0))
    assert (o == np.tile(np.arange(64, dtype=np.float32) / 2, 64)).all()
    # ring of 128 at position 200, q = 0, sink -inf: equal weights over slots 0..127 (mean 63.5)
    cv2 = np.repeat(np.array([f16_entier(s) for s in range(128)], np.uint16), dkv)
    p = O.attention_gpt_oss(200, 128)
    assert (p.debut, p.fin) == (73, 201)
    o = O.attention(np.zeros(64 * 64, np.float32), np.full(128 * dkv, UN16, np.uint16), cv2,
                    np.full(64, -np.inf, np.float32), p)
    assert np.abs(o - 63.5).max() <= 1e-4
    # 4096 positions, v = position mod 2048: mean 1023.5
    cv3 = np.repeat(np.array([f16_entier(j % 2048) for j in range(4096)], np.uint16), dkv)
    o = O.attention(np.zeros(64 * 64, np.float32), np.full(4096 * dkv, UN16, np.uint16), cv3,
                    np.full(64, -np.inf, np.float32), O.attention_gpt_oss(4095, 0))
    assert np.abs(o - 1023.5).max() <= 1e-2


def attention_f64(q, ck, cv, puits, p):
    """ops.rs:87-118 in f64 over the f16 cache values, head by head."""
    dkv = p.tetes_kv * 64
    K = ck.view(np.float16).astype(np.float64)
    V = cv.view(np.float16).astype(np.float64)
    out = np.zeros(64 * p.tetes)
    for h in range(p.tetes):
        hk = h // (p.tetes // p.tetes_kv)
        pos = np.arange(p.debut, p.fin)
        cases = pos % p.anneau if p.anneau else pos
        ks = K.reshape(-1, dkv)[cases, hk * 64:(hk + 1) * 64]
        vs = V.reshape(-1, dkv)[cases, hk * 64:(hk + 1) * 64]
        s = ks @ q[h * 64:(h + 1) * 64].astype(np.float64) * p.echelle
        m = max(s.max() if s.size else -np.inf, float(puits[h]))
        e = np.exp(s - m)
        z = e.sum() + math.exp(float(puits[h]) - m)
        out[h * 64:(h + 1) * 64] = (e[:, None] * vs).sum(axis=0) / z
    return out


@pytest.mark.parametrize("position,fenetre", [(5, 0), (300, 128), (1000, 0)])
def test_attention_random_against_f64(position, fenetre):
    rng = np.random.default_rng(position)
    p = O.attention_gpt_oss(position, fenetre)
    cases = fenetre if fenetre else position + 1
    q = rng.standard_normal(64 * 64).astype(np.float32)
    ck = (rng.standard_normal(cases * 512) * 0.5).astype(np.float16).view(np.uint16)
    cv = rng.standard_normal(cases * 512).astype(np.float16).view(np.uint16)
    puits = rng.standard_normal(64).astype(np.float32)
    o = O.attention(q, ck, cv, puits, p)
    ref = attention_f64(q, ck, cv, puits, p)
    assert np.abs(o - ref).max() <= 1e-5 * np.abs(ref).max()


def test_argmax_ties_and_nan():
    # tests/passe.rs:296-302
    v = np.zeros(100_000, np.float32)
    v[0] = np.nan
    v[70_000] = 5.0
    v[12_345] = 5.0
    assert O.argmax(v) == 12_345
    assert O.argmax(np.full(10, np.nan, np.float32)) == 0xFFFFFFFF
    assert O.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
