"""The rest of the layer step on the GPU (csrc/passe.hip) through the C-ABI, against the oracle
(oracle/passe.c, the reference's operation order) and the reference's own fixtures
(moteur/crates/trc-noyaux/tests/passe.rs):
- gemv_q8_0: exact on the integer fixture (37 x 96 and 2880 x 4096, bias), and bit for bit equal
  to the oracle on random data (same lane order and butterfly), rows not a multiple of 32;
- ligne_q8_0 exact; ecrire_kv bit for bit (the fixture's ties, subnormals, overflow, its slot);
- rmsnorm bit for bit against the oracle (same f64 tree), in place too;
- rope_yarn within 1e-6 of the oracle (f64 libm functions may differ in the last bit), and the
  fixture's closed forms;
- attention: the fixture's three cases, random heads within 1e-6 of f64 and 3e-6 of the oracle's
  reference-order result;
- argmax: the fixture's tie and NaN, random vectors.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle_ffi as O  # noqa: E402
from gpu_outils import dev, hote, vue, zeros  # noqa: E402
from test_oracle_passe import Alea, attention_f64, f16_entier, q8_0_entier, UN16  # noqa: E402
from troncons_amd.noyaux import Noyaux, ParamsAttention, ParamsRope  # noqa: E402


@pytest.fixture(scope="module")
def k():
    assert torch.cuda.is_available()
    return Noyaux.charger()


def _q8(k, o, x, biais, r, c):
    y = zeros(4 * r)
    k.gemv_q8_0(vue(dev(o)), vue(dev(x)), vue(dev(biais)) if biais is not None else None, vue(y), r, c)
    return hote(y, np.float32)


@pytest.mark.parametrize("r,c", [(37, 96), (2880, 4096)])
def test_gemv_q8_0_integer_exact(k, r, c):
    print(f"gemv_q8_0 exact {r}x{c}", flush=True)
    o, x, biais, attendu = q8_0_entier(Alea(31), r, c)
    assert (_q8(k, o, x, biais, r, c) == attendu.astype(np.float32)).all()


@pytest.mark.parametrize("r,c", [(100, 2880), (4096, 2880), (2880, 4096)])
def test_gemv_q8_0_bit_exact_against_oracle(k, r, c):
    print(f"gemv_q8_0 random {r}x{c}", flush=True)
    rng = np.random.default_rng(r + c)
    nb = c // 32
    d = (rng.standard_normal(r * nb) * 0.01).astype(np.float16)
    q = rng.integers(-128, 128, size=(r * nb, 32)).astype(np.int8)
    o = np.concatenate([d.view(np.uint8).reshape(-1, 2), q.view(np.uint8)], axis=1).ravel()
    x = rng.standard_normal(c).astype(np.float32)
    b = rng.standard_normal(r).astype(np.float32)
    ref = O.gemv_q8_0(o, x, b, r, c)
    got = _q8(k, o, x, b, r, c)
    assert (got.view(np.uint32) == ref.view(np.uint32)).all()
    assert (_q8(k, o, x, None, r, c).view(np.uint32) == O.gemv_q8_0(o, x, None, r, c).view(np.uint32)).all()


def test_gemv_q8_0_unaligned_matrix_and_last_block(k):
    # a matrix starting 2 bytes past a 4-byte boundary (the contract allows any even address), with
    # the last block's window reaching past the matrix end on a view that ends there
    rng = np.random.default_rng(12)
    for r, c in ((33, 64), (7, 2880)):
        nb = c // 32
        d = (rng.standard_normal(r * nb) * 0.05).astype(np.float16)
        q = rng.integers(-128, 128, size=(r * nb, 32)).astype(np.int8)
        o = np.concatenate([d.view(np.uint8).reshape(-1, 2), q.view(np.uint8)], axis=1).ravel()
        x = rng.standard_normal(c).astype(np.float32)
        base = zeros(o.size + 2)
        base[2:].copy_(torch.from_numpy(o.copy()).to(base.device))
        y = zeros(4 * r)
        k.gemv_q8_0(vue(base, 2, o.size), vue(dev(x)), None, vue(y), r, c)
        assert (hote(y, np.float32).view(np.uint32) == O.gemv_q8_0(o, x, None, r, c).view(np.uint32)).all()


def test_gemv_q8_0_wide_rows_read_x_from_global_memory(k):
    """Past 16384 columns x does not fit the LDS staging: the short launch reads it from global
    memory, with the same values."""
    rng = np.random.default_rng(16416)
    r, c = 40, 16416
    nb = c // 32
    d = (rng.standard_normal(r * nb) * 0.05).astype(np.float16)
    q = rng.integers(-128, 128, size=(r * nb, 32)).astype(np.int8)
    o = np.concatenate([d.view(np.uint8).reshape(-1, 2), q.view(np.uint8)], axis=1).ravel()
    x = rng.standard_normal(c).astype(np.float32)
    y = zeros(4 * r)
    k.gemv_q8_0(vue(dev(o)), vue(dev(x)), None, vue(y), r, c)
    assert (hote(y, np.float32).view(np.uint32) == O.gemv_q8_0(o, x, None, r, c).view(np.uint32)).all()


@pytest.mark.parametrize("r,c,decalage", [(32769, 96, 0), (32770, 96, 2), (40000, 2880, 0), (32800, 2880, 2)])
def test_gemv_q8_0_large_matrices(k, r, c, decalage):
    """From 32768 rows the launch takes four rows per half-wavefront (the output head's kernel):
    bit-identical to the oracle, with the matrix at a 4-byte boundary or 2 bytes past one, and
    ending 2 bytes into a dword (32769 x 96 aligned, 32770 x 96 offset) or on one."""
    rng = np.random.default_rng(r + decalage)
    nb = c // 32
    d = (rng.standard_normal(r * nb) * 0.05).astype(np.float16)
    q = rng.integers(-128, 128, size=(r * nb, 32)).astype(np.int8)
    o = np.concatenate([d.view(np.uint8).reshape(-1, 2), q.view(np.uint8)], axis=1).ravel()
    x = rng.standard_normal(c).astype(np.float32)
    base = zeros(o.size + decalage)
    base[decalage:].copy_(torch.from_numpy(o.copy()).to(base.device))
    b = rng.standard_normal(r).astype(np.float32)
    y = zeros(4 * r)
    k.gemv_q8_0(vue(base, decalage, o.size), vue(dev(x)), vue(dev(b)), vue(y), r, c)
    assert (hote(y, np.float32).view(np.uint32) == O.gemv_q8_0(o, x, b, r, c).view(np.uint32)).all()


def test_ligne_q8_0_exact(k):
    a = Alea(7)
    lignes, c = 5, 64
    o = np.zeros(lignes * 2 * 34, np.uint8)
    for bl in range(lignes * 2):
        o[bl * 34:bl * 34 + 2] = np.frombuffer(np.uint16((a.entre(-14, 15) + 15) << 10).tobytes(), np.uint8)
        o[bl * 34 + 2:bl * 34 + 34] = np.array([a.entre(-128, 127) for _ in range(32)]).astype(np.int8).view(np.uint8)
    w = dev(o)
    for l in range(lignes):
        y = zeros(4 * c)
        k.ligne_q8_0(vue(w), l, c, vue(y))
        assert (hote(y, np.float32) == O.ligne_q8_0(o, l, c)).all(), l


def test_ecrire_kv_bit_exact(k):
    kk = np.array([1.0, -2.5, 0.0, 65504.0, 1.0 + 2.0 ** -11, 1.0 + 3.0 * 2.0 ** -11, -0.0, 6.1035156e-5], np.float32)
    ck, cv = zeros(2 * 8 * 3), zeros(2 * 8 * 3)
    kd = dev(kk)
    k.ecrire_kv(vue(kd), vue(kd), vue(ck), vue(cv), 8, 2)
    got = hote(ck, np.uint16)
    assert list(got[16:]) == [0x3C00, 0xC100, 0x0000, 0x7BFF, 0x3C00, 0x3C02, 0x8000, 0x0400]
    assert (got[:16] == 0).all()
    # every regime: normal, f16 subnormal, overflow to inf, ties
    rng = np.random.default_rng(9)
    dkv = 512
    v = np.concatenate([rng.standard_normal(200) * 2.0 ** rng.integers(-26, 17, 200),
                        rng.uniform(65000, 66000, 56), np.float16(rng.standard_normal(256)).astype(np.float64) * (1 + 2 ** -11)])
    v = v.astype(np.float32)[:dkv]
    w = -v[::-1].copy()
    ck, cv = zeros(2 * dkv * 4), zeros(2 * dkv * 4)
    k.ecrire_kv(vue(dev(v)), vue(dev(w)), vue(ck), vue(cv), dkv, 3)
    rk, rv = O.ecrire_kv(v, w, np.zeros(dkv * 4, np.uint16), np.zeros(dkv * 4, np.uint16), dkv, 3)
    assert (hote(ck, np.uint16) == rk).all() and (hote(cv, np.uint16) == rv).all()


def test_rmsnorm_bit_exact_and_in_place(k):
    a = Alea(11)
    n = 2880
    x = np.array([a.entre(-1000, 1000) / 37.0 for _ in range(2 * n)], np.float32)
    w = np.array([a.entre(1, 300) / 100.0 for _ in range(n)], np.float32)
    ref = O.rmsnorm(x, w, n, 2, 1e-5)
    xd, wd, y = dev(x), dev(w), zeros(8 * n)
    k.rmsnorm(vue(xd), vue(wd), vue(y), n, 2, 1e-5)
    assert (hote(y, np.float32).view(np.uint32) == ref.view(np.uint32)).all()
    k.rmsnorm(vue(xd), vue(wd), vue(xd), n, 2, 1e-5)  # y = x
    assert (hote(xd, np.float32).view(np.uint32) == ref.view(np.uint32)).all()
    rng = np.random.default_rng(4)
    # up to 4096 a thread keeps its values in registers; past it the loop form (5000, 8191)
    for n2, l2 in ((64, 64), (4096, 3), (1000, 1), (5000, 2), (8191, 1)):
        x2 = rng.standard_normal(n2 * l2).astype(np.float32)
        w2 = rng.standard_normal(n2).astype(np.float32)
        y2 = zeros(4 * n2 * l2)
        k.rmsnorm(vue(dev(x2)), vue(dev(w2)), vue(y2), n2, l2, 1e-6)
        assert (hote(y2, np.float32).view(np.uint32) == O.rmsnorm(x2, w2, n2, l2, 1e-6).view(np.uint32)).all()


def _rope(k, q, kk, tq, tk, pos, p):
    qd, kd = dev(q), dev(kk)
    k.rope_yarn(vue(qd), vue(kd), tq, tk, pos, p)
    return hote(qd, np.float32), hote(kd, np.float32)


def test_rope_yarn_against_oracle(k):
    a = Alea(11)
    q = np.array([a.entre(-500, 500) / 64.0 for _ in range(64 * 64)], np.float32)
    kk = np.array([a.entre(-500, 500) / 64.0 for _ in range(8 * 64)], np.float32)
    m = 0.1 * np.log(32.0) + 1.0
    gq, _ = _rope(k, q, kk, 64, 8, 0, ParamsRope.gpt_oss())
    assert np.abs(gq - q.astype(np.float64) * m).max() <= 1e-6 * np.abs(q * m).max()
    for pos in (1, 1000, 131071):
        for var in (0, 1):
            p = ParamsRope.gpt_oss(variante=var)
            gq, gk = _rope(k, q, kk, 64, 8, pos, p)
            rq, rk = O.rope_yarn(q, kk, 64, 8, pos, O.rope_gpt_oss(variante=var))
            assert np.abs(gq - rq).max() <= 1e-6 * np.abs(rq).max() and np.abs(gk - rk).max() <= 1e-6 * np.abs(rk).max()
            assert (gq == rq).mean() > 0.99, (pos, var)
    # factor 1 (plain RoPE) and another head size
    gq, gk = _rope(k, q[:128], kk[:128], 1, 1, 1000, ParamsRope.gpt_oss(facteur=1.0, dim_tete=128))
    rq, rk = O.rope_yarn(q[:128], kk[:128], 1, 1, 1000, O.rope_gpt_oss(facteur=1.0, dim_tete=128))
    assert np.abs(gq - rq).max() <= 1e-6 * np.abs(rq).max() and np.abs(gk - rk).max() <= 1e-6 * np.abs(rk).max()


def _attention(k, q, ck, cv, puits, p):
    s = zeros(4 * 64 * p.tetes)
    k.attention(vue(dev(q)), vue(dev(ck)), vue(dev(cv)), vue(dev(puits)), vue(s), p)
    return hote(s, np.float32)


def test_attention_fixture_cases(k):
    dkv = 8 * 64
    ck = np.full(dkv, UN16, np.uint16)
    cv = np.array([f16_entier(t % 64) for t in range(dkv)], np.uint16)
    o = _attention(k, np.zeros(64 * 64, np.float32), ck, cv, np.zeros(64, np.float32), ParamsAttention.gpt_oss(0, 0))
    assert (o == np.tile(np.arange(64, dtype=np.float32) / 2, 64)).all()
    cv2 = np.repeat(np.array([f16_entier(s) for s in range(128)], np.uint16), dkv)
    p = ParamsAttention.gpt_oss(200, 128)
    o = _attention(k, np.zeros(64 * 64, np.float32), np.full(128 * dkv, UN16, np.uint16), cv2,
                   np.full(64, -np.inf, np.float32), p)
    assert np.abs(o - 63.5).max() <= 1e-4
    cv3 = np.repeat(np.array([f16_entier(j % 2048) for j in range(4096)], np.uint16), dkv)
    o = _attention(k, np.zeros(64 * 64, np.float32), np.full(4096 * dkv, UN16, np.uint16), cv3,
                   np.full(64, -np.inf, np.float32), ParamsAttention.gpt_oss(4095, 0))
    assert np.abs(o - 1023.5).max() <= 1e-2


@pytest.mark.parametrize("position,fenetre", [(0, 0), (5, 0), (300, 128), (2047, 0), (8191, 0)])
def test_attention_random_against_oracle(k, position, fenetre):
    print(f"attention position {position} window {fenetre}", flush=True)
    rng = np.random.default_rng(position + 7)
    p = ParamsAttention.gpt_oss(position, fenetre)
    po = O.attention_gpt_oss(position, fenetre)
    cases = fenetre if fenetre else position + 1
    q = rng.standard_normal(64 * 64).astype(np.float32)
    ck = (rng.standard_normal(cases * 512) * 0.5).astype(np.float16).view(np.uint16)
    cv = rng.standard_normal(cases * 512).astype(np.float16).view(np.uint16)
    puits = rng.standard_normal(64).astype(np.float32)
    got = _attention(k, q, ck, cv, puits, p)
    ref = O.attention(q, ck, cv, puits, po)
    ref64 = attention_f64(q, ck, cv, puits, po)
    # The one-pass running softmax adds its terms in 64-position chunks, the reference in four
    # chains of every fourth position: it lands closer to f64 (at 8192 positions 2.4e-7 of max|out|
    # against the reference order's 1.3e-6), and the two f32 results differ by about their sum.
    assert np.abs(got - ref64).max() <= 1e-6 * np.abs(ref64).max()
    assert np.abs(got - ref).max() <= 3e-6 * np.abs(ref).max()


def test_attention_first_chunk_of_minus_inf_scores(k):
    """Positions 0..63 (the first chunk of the first wavefront) hold keys with a -inf component
    against a positive query component: their scores are -inf and their weights 0, since the
    reference's maximum includes the sink before any exponential (passe.cuh:306-371). The output
    stays finite and meets the random-head tolerances."""
    position = 300
    rng = np.random.default_rng(17)
    p = ParamsAttention.gpt_oss(position, 0)
    po = O.attention_gpt_oss(position, 0)
    q = rng.standard_normal(64 * 64).astype(np.float32)
    q.reshape(64, 64)[:, 5] = np.abs(q.reshape(64, 64)[:, 5]) + 0.25
    ck = (rng.standard_normal((position + 1) * 512) * 0.5).astype(np.float16)
    ck.reshape(position + 1, 8, 64)[:64, :, 5] = -np.inf
    ck = ck.view(np.uint16)
    cv = rng.standard_normal((position + 1) * 512).astype(np.float16).view(np.uint16)
    puits = rng.standard_normal(64).astype(np.float32)
    got = _attention(k, q, ck, cv, puits, p)
    assert np.isfinite(got).all()
    ref = O.attention(q, ck, cv, puits, po)
    ref64 = attention_f64(q, ck, cv, puits, po)
    assert np.isfinite(ref).all() and np.isfinite(ref64).all()
    assert np.abs(got - ref64).max() <= 1e-6 * np.abs(ref64).max()
    assert np.abs(got - ref).max() <= 3e-6 * np.abs(ref).max()


def test_argmax_ties_nan_and_random(k):
    v = np.zeros(100_000, np.float32)
    v[0] = np.nan
    v[70_000] = 5.0
    v[12_345] = 5.0
    s = zeros(4)
    k.argmax(vue(dev(v)), v.size, vue(s))
    assert hote(s, np.uint32)[0] == 12_345
    k.argmax(vue(dev(np.full(33, np.nan, np.float32))), 33, vue(s))
    assert hote(s, np.uint32)[0] == 0xFFFFFFFF
    rng = np.random.default_rng(2)
    for n in (1, 1000, 201_088):
        r = rng.integers(-50, 50, n).astype(np.float32)
        k.argmax(vue(dev(r)), n, vue(s))
        assert hote(s, np.uint32)[0] == O.argmax(r) == int(np.argmax(r))


def test_usage_errors_are_refused(k):
    from troncons_amd.noyaux import ErreurUsage
    with pytest.raises(ErreurUsage):
        k.gemv_q8_0(vue(zeros(34)), vue(zeros(128)), None, vue(zeros(4)), 1, 48)  # columns % 32
    with pytest.raises(ErreurUsage):
        k.attention(vue(zeros(4 * 64 * 64)), vue(zeros(1024)), vue(zeros(1024)), vue(zeros(256)), vue(zeros(4 * 64 * 64)),
                    ParamsAttention.gpt_oss(8192, 0))  # 8193 positions
    with pytest.raises(ErreurUsage):
        k.rope_yarn(vue(zeros(256)), vue(zeros(256)), 1, 1, 0, ParamsRope.gpt_oss(variante=2))


@pytest.mark.parametrize("anneau,representable", [(0, True), (128, True), (0, False)])
def test_kv_f32_equals_f16_path_on_representable_values(k, anneau, representable):
    """tests/passe.rs:395-433: with keys and values m / 256, |m| <= 1024 (exact in f16), the f32
    cache path (ecrire_kv_f32 + attention_kvf32) gives the f16 path's outputs bit for bit, on a full
    cache and on a 128-slot ring at position 300; values 1e-3 off that grid make the paths differ."""
    dkv, position = 8 * 64, 300
    rng = np.random.default_rng(20261016 + anneau + int(representable))
    cases = anneau if anneau else position + 1
    c16k, c16v = zeros(2 * cases * dkv), zeros(2 * cases * dkv)
    c32k, c32v = zeros(4 * cases * dkv), zeros(4 * cases * dkv)
    for p in range(position + 1):
        kv = [(rng.integers(-1024, 1025, dkv) / 256.0 + (0.0 if representable else 1e-3)).astype(np.float32)
              for _ in range(2)]
        kd, vd = dev(kv[0]), dev(kv[1])
        case = ParamsAttention.case(p, anneau)
        k.ecrire_kv(vue(kd), vue(vd), vue(c16k), vue(c16v), dkv, case)
        k.ecrire_kv_f32(vue(kd), vue(vd), vue(c32k), vue(c32v), dkv, case)
    q = (rng.integers(-1000, 1001, 64 * 64) / 333.0).astype(np.float32)
    puits = (rng.integers(-300, 301, 64) / 100.0).astype(np.float32)
    pa = ParamsAttention.gpt_oss(position, anneau)
    s16, s32 = zeros(4 * 64 * 64), zeros(4 * 64 * 64)
    k.attention(vue(dev(q)), vue(c16k), vue(c16v), vue(dev(puits)), vue(s16), pa)
    k.attention_kvf32(vue(dev(q)), vue(c32k), vue(c32v), vue(dev(puits)), vue(s32), pa)
    differents = int((hote(s16, np.uint32) != hote(s32, np.uint32)).sum())
    if representable:
        assert differents == 0
    else:
        assert differents > 0
