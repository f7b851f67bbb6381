"""Pins the CPU oracle's rANS codec (oracle/rans.c) against the reference's own known answers and
against hand-derived closed forms — never against a re-typed copy of the same formula.

Reference tests followed: moteur/crates/trc-noyaux/src/abi.rs:384-406 (LUT known answers),
moteur/crates/trc-codec/tests/rans.rs:115-255 (round trips, breaks, refusals).
"""
import numpy as np
import pytest

import oracle_ffi as O


# --------------------------------------------------------------------------------------- LUT

def test_lut_known_answers_abi_rs_384():
    f = np.zeros(256, np.uint16)
    f[3], f[200] = 4000, 96
    _, l = O.lut(f)
    assert l[0] == 3 | (3999 << 8)
    assert l[3999] == 3 | (3999 << 8) | (3999 << 20)
    assert l[4000] == 200 | (95 << 8)
    assert l[4095] == 200 | (95 << 8) | (95 << 20)
    f[3] = 3999  # break: wrong sum is refused
    assert O.lut(f) is None


def test_lut_single_symbol_full_frequency_abi_rs_399():
    f = np.zeros(256, np.uint16)
    f[7] = 4096
    _, l = O.lut(f)
    assert l[4095] == 7 | (4095 << 8) | (4095 << 20)


def test_depuis_frequences_refusals_rans_tests_245():
    f = np.zeros(16, np.uint16)
    f[0] = 4095
    assert O.lut(f, 2) is None
    f[1] = 1
    assert O.lut(f, 2) is not None


# ------------------------------------------------------------------------------ normalisation

def test_all_zero_counts_give_symbol_0_everything_rans_tests_253():
    f = O.table_depuis_comptes(np.zeros(256, np.uint64))
    assert f[0] == 4096 and f.sum() == 4096


def _c(vals, n=256):
    c = np.zeros(n, np.uint64)
    c[: len(vals)] = vals
    return c


def test_normalisation_hand_derived_geometry1():
    # 3 equal counts: round(4096/3) = 1365 each, sum 4095; the +1 goes to the first symbol of the
    # stable decreasing order (all equal -> index 0).
    assert list(O.table_depuis_comptes(_c([1, 1, 1]))[:3]) == [1366, 1365, 1365]
    # 6 equal counts: round(682.67) = 683 each, sum 4098; -1 to symbols 0 then 1.
    assert list(O.table_depuis_comptes(_c([5] * 6))[:6]) == [682, 682, 683, 683, 683, 683]
    # (1, 1e6): max(1, round(0.004)) = 1 and round(4095.996) = 4096 -> sum 4097 -> 4095.
    assert list(O.table_depuis_comptes(_c([1, 1_000_000]))[:2]) == [1, 4095]
    # (1, 1, 1e9): the walk wraps around: 4096 -> 4095, skip the two 1s, -> 4094.
    assert list(O.table_depuis_comptes(_c([1, 1, 10**9]))[:3]) == [1, 1, 4094]
    # exact proportions are kept
    f = O.table_depuis_comptes(np.full(256, 7, np.uint64))
    assert (f == 16).all()


def test_normalisation_hand_derived_geometry2():
    # geometry 2 gives the whole gap to the LAST maximal symbol (Iterator::max_by_key).
    assert list(O.table_depuis_comptes(_c([1, 1, 1], 16), 2)[:3]) == [1365, 1365, 1366]
    assert list(O.table_depuis_comptes(_c([5] * 6, 16), 2)[:6]) == [683, 683, 683, 683, 683, 681]


# ------------------------------------------------------------------- stream: closed forms

def _table_2048():
    f = np.zeros(256, np.uint16)
    f[0] = f[1] = 2048
    return f


def test_closed_form_states_one_macro_step():
    """Symbols 0/1 with f = 2048 cost exactly one bit and never renormalise: encoding the lane's
    bytes s0..s3 in reverse order from x = L gives x = 2^20 + 2048 * (s0 + 2 s1 + 4 s2 + 8 s3)."""
    rng = np.random.default_rng(1)
    src = rng.integers(0, 2, 128).astype(np.uint8)
    b = O.coder(src, _table_2048())
    hdr = np.frombuffer(b[:16], np.uint32)
    assert hdr[0] == 128 and (hdr[1] & 0xFFFF) == 256 and ((hdr[1] >> 16) & 0xFF) == 1 and hdr[2] == 1 and hdr[3] == 0
    assert len(b) == 160  # 16 + 4 + 128 = 148, padded to 16
    starts = np.frombuffer(b[16:20], np.uint32)
    states = np.frombuffer(b[20:148], np.uint32)
    assert starts[0] == 0
    s = src.reshape(32, 4).astype(np.uint64)  # lane l -> bytes 4l .. 4l+3
    attendu = (1 << 20) + 2048 * (s[:, 0] + 2 * s[:, 1] + 4 * s[:, 2] + 8 * s[:, 3])
    assert (states == attendu).all()
    _, lut = O.lut(_table_2048())
    dec, bil = O.decoder(b, lut)
    assert (dec == src).all() and bil.voies_hors_l == 0 and bil.tuiles_mots_faux == 0


def _table_rare():
    f = np.zeros(256, np.uint16)
    f[0], f[1] = 1, 4095  # c[0] = 0, c[1] = 1
    return f


def test_closed_form_word_order():
    """Hand-derived stream (see derivation below): lanes 0 and 1 each push one word at sub-step 0,
    every other lane encodes four common symbols. Words must appear in lane order.

    lane 0, bytes [0,1,1,0]: L -> (rare) 2^28 -> (common) 268501009 -> (common) 268566578 ->
        (rare: 268566578 >= 2^20, push 268566578 mod 2^16 = 50, x = 4098) 4098*4096 = 16785408
    lane 1, bytes [0,0,1,1]: L -> 65553 -> 65570 -> (rare) 65570*4096 -> (rare: push 8192,
        x = 4098) 16785408
    other lanes [1,1,1,1]: each common symbol adds 17 near L: 65604.
    Encoder stack (k = 0, lanes 31..0): [8192, 50], reversed -> words [50, 8192]."""
    src = np.ones(128, np.uint8)
    src[0:4] = [0, 1, 1, 0]
    src[4:8] = [0, 0, 1, 1]
    for N in (256, 1):
        for rep in (1, 2):
            s = np.tile(src, rep)
            b = O.coder(s, _table_rare(), N=N)
            hdr = np.frombuffer(b[:16], np.uint32)
            T = hdr[2]
            assert T == (rep if N == 1 else 1)
            W = hdr[3]
            starts = np.frombuffer(b[16:16 + 4 * T], np.uint32)
            states = np.frombuffer(b[16 + 4 * T:16 + 132 * T], np.uint32)
            words = np.frombuffer(b[16 + 132 * T:16 + 132 * T + 2 * W], np.uint16)
            if N == 1:
                assert list(starts) == [2 * t for t in range(rep)]
                tile_states = np.array([16785408, 16785408] + [65604] * 30, np.uint32)
                assert (states == np.tile(tile_states, rep)).all()
                assert list(words) == [50, 8192] * rep
            _, lut = O.lut(_table_rare())
            dec, bil = O.decoder(b, lut)
            assert (dec == s).all() and bil.voies_hors_l == 0 and bil.tuiles_mots_faux == 0


# ---------------------------------------------------------------- stream: refusals and breaks

def _geom(rng, n, p, size):
    u = rng.random(size)
    return np.minimum((np.log1p(-u) / np.log1p(-p)).astype(np.int64), n - 1)


def _source(rng, n):
    return (_geom(rng, 16, 0.3, n) | (_geom(rng, 16, 0.25, n) << 4)).astype(np.uint8)


def _tables_par_classe(src, kappa):
    c = np.zeros((3, 256), np.uint64)
    blk = np.arange(src.size) // 16
    k = np.where(blk < kappa.size, kappa[np.minimum(blk, kappa.size - 1)], 0)
    for cl in range(3):
        c[cl] = np.bincount(src[k == cl], minlength=256)
    return np.stack([O.table_depuis_comptes(c[i]) for i in range(3)])


@pytest.mark.parametrize("n_blocs", [8, 1000, 8 * 2025])
@pytest.mark.parametrize("N", [256, 32, 7])
def test_round_trip_per_lane_context(n_blocs, N):
    rng = np.random.default_rng(n_blocs + N)
    src = _source(rng, 16 * n_blocs)
    kappa = np.array([0, 1, 1, 2], np.uint8)[rng.integers(0, 4, n_blocs)]
    src[np.repeat(kappa, 16) == 2] &= 0x33
    t = _tables_par_classe(src, kappa)
    luts = np.concatenate([O.lut(t[i])[1] for i in range(3)])
    b = O.coder(src, t, kappa=kappa, N=N)
    dec, bil = O.decoder(b, luts, kappa=kappa)
    assert (dec == src).all()
    assert bil.voies_hors_l == 0 and bil.tuiles_mots_faux == 0


def test_breaks_are_seen_rans_tests_190():
    rng = np.random.default_rng(5)
    n_blocs = 4000
    src = _source(rng, 16 * n_blocs)
    kappa = np.array([0, 1, 1, 2], np.uint8)[rng.integers(0, 4, n_blocs)]
    t = _tables_par_classe(src, kappa)
    luts = np.concatenate([O.lut(t[i])[1] for i in range(3)])
    b = O.coder(src, t, kappa=kappa)
    dec, bil = O.decoder(b, luts, kappa=kappa)
    assert (dec == src).all() and bil.voies_hors_l == 0

    # 1. two frequencies swapped in the class-1 table
    f1 = t[1].copy()
    ordre = np.argsort(-f1.astype(np.int64), kind="stable")
    f1[ordre[0]], f1[ordre[1]] = f1[ordre[1]], f1[ordre[0]]
    lf = np.concatenate([O.lut(t[0])[1], O.lut(f1)[1], O.lut(t[2])[1]])
    d, bil = O.decoder(b, lf, kappa=kappa)
    assert (d != src).any() and bil.voies_hors_l > 0

    f = O.flux_lire(b)
    T, W = f.T, f.W
    mots0 = 16 + 132 * T
    # 2. a word flipped, then a state flipped
    q = bytearray(b)
    k = mots0 + 2 * (W // 2)
    q[k + 1] ^= 0x01
    d, bil = O.decoder(bytes(q), luts, kappa=kappa)
    assert (d != src).any() and (bil.voies_hors_l > 0 or bil.tuiles_mots_faux > 0)
    q = bytearray(b)
    q[16 + 4 * T + 4 * 5] ^= 1
    d, bil = O.decoder(bytes(q), luts, kappa=kappa)
    assert (d != src).any() and bil.voies_hors_l > 0
    # one extra word at the end of the last tile: output and lanes stay right; only the word-count
    # check sees it
    body = bytearray(b[:mots0 + 2 * W]) + bytes([0xCD, 0xAB])
    body[12:16] = np.uint32(W + 1).tobytes()
    body += bytes((-len(body)) % 16)
    d, bil = O.decoder(bytes(body), luts, kappa=kappa)
    assert (d == src).all() and bil.voies_hors_l == 0 and bil.tuiles_mots_faux == 1

    # 3. corrupted header fields are refused; truncation is refused
    for pos in (0, 7, 8, 6):
        q = bytearray(b)
        q[pos] ^= 0x41
        assert O.flux_lire(bytes(q)) is None
    assert O.flux_lire(b[:-64]) is None
