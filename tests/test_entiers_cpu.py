"""Host build of the integer helpers the kernels share (troncons_amd/csrc/entiers.hpp), compiled with
g++ and checked on the CPU:

- Diviseur (division by an invariant through a multiply-high, Granlund & Montgomery 1994) against the
  plain quotient for every divisor the slot decoders can meet (blocks per row, 1 .. 4096) and many
  more up to 2^31, on numerators chosen where a wrong multiplier or shift fails first: 0, 2^32 - 1,
  every multiple of the divisor near the top of the range, its neighbours, and random values.
- elargir_u64, the widening of two `readfirstlane` results (int) into a 64-bit address: a low word
  with bit 31 set must not spill into the high word (a plain int -> uint64 conversion would
  sign-extend it), and a high word with bit 31 set must survive.
"""
from __future__ import annotations

import pathlib
import shutil
import subprocess

import pytest

RACINE = pathlib.Path(__file__).resolve().parents[1]

PROGRAMME = r"""
#include <cstdio>
#include <cstdint>
#include <random>
#include <vector>
#include "entiers.hpp"

static int echecs = 0;
static void verifier(uint32_t n, uint32_t d) {
    const trc::Diviseur q = trc::Diviseur::de(d);
    if (q.quotient(n) != n / d) {
        if (echecs++ < 10) std::printf("faux: %u / %u = %u, obtenu %u\n", n, d, n / d, q.quotient(n));
    }
}

int main() {
    std::mt19937_64 g(2026);
    std::vector<uint32_t> diviseurs;
    for (uint32_t d = 1; d <= 4096; ++d) diviseurs.push_back(d);
    for (uint32_t k = 12; k <= 31; ++k) {
        const uint32_t p = 1u << k;
        diviseurs.push_back(p - 1u);
        diviseurs.push_back(p);
        diviseurs.push_back(p + 1u);
    }
    for (int i = 0; i < 2000; ++i) diviseurs.push_back(1u + uint32_t(g() % 0x7FFFFFFFu));
    for (uint32_t d : diviseurs) {
        verifier(0u, d);
        verifier(0xFFFFFFFFu, d);
        verifier(d - 1u, d);
        verifier(d, d);
        const uint32_t haut = 0xFFFFFFFFu / d;
        for (uint32_t k = 0; k < 4 && k <= haut; ++k) {
            const uint64_t m = uint64_t(haut - k) * d;
            verifier(uint32_t(m), d);
            if (m > 0) verifier(uint32_t(m - 1u), d);
            if (m + d - 1u <= 0xFFFFFFFFull) verifier(uint32_t(m + d - 1u), d);
        }
        for (int i = 0; i < 64; ++i) verifier(uint32_t(g()), d);
    }
    // widening of readfirstlane results
    const int bas = int(0x80000010u), haut = int(0x00007FFFu);
    if (trc::elargir_u64(bas, haut) != 0x00007FFF80000010ull) { std::printf("elargir bas\n"); ++echecs; }
    if (trc::elargir_u64(int(0x0000ABCDu), int(0xFFFF8000u)) != 0xFFFF80000000ABCDull) { std::printf("elargir haut\n"); ++echecs; }
    if (trc::elargir_u64(-1, 0) != 0x00000000FFFFFFFFull) { std::printf("elargir -1\n"); ++echecs; }
    // what the helper guards against: the int itself widened sign-extends
    if ((uint64_t(int64_t(bas)) >> 32) != 0xFFFFFFFFull) { std::printf("temoin\n"); ++echecs; }
    std::printf("%d\n", echecs);
    return echecs == 0 ? 0 : 1;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ absent")
def test_integer_helpers_on_the_host(tmp_path):
    src = tmp_path / "entiers_hote.cpp"
    src.write_text(PROGRAMME)
    exe = tmp_path / "entiers_hote"
    subprocess.run(["g++", "-O2", "-std=c++17", "-Wall", "-Werror", "-I", str(RACINE / "troncons_amd" / "csrc"),
                    str(src), "-o", str(exe)], check=True, capture_output=True, timeout=120)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().splitlines()[-1] == "0"
