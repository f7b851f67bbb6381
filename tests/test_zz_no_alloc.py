"""The allocation-free MoE layer step (trc_couche_moe_fusionnee_sans_alloc) against the allocating one
(trc_couche_moe_fusionnee), through the C-ABI: same routing, weights and residual bits, on two calls
in a row, the second on a smaller layer (the static scratch keeps the first call's contents), and a
step larger than the scratch refused before any launch."""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle_ffi as O  # noqa: E402
from gpu_outils import dev, hote, vue, zeros  # noqa: E402
from troncons_amd import codeur, fusion  # noqa: E402
from troncons_amd.noyaux import DimsExpert, ErreurUsage  # noqa: E402


class Couche:
    def __init__(self, fz, graine, E, dims, N):
        self.c = codeur.CoucheSynthetique(graine, 0, E, dims, N_delta=N[0], N_codes=N[1])
        freqs = self.c.freqs()
        self.luts = dev(O.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)]))
        self.parts = [dev(self.c.partie(e)) for e in range(E)]
        self.table = dev(np.array([p.data_ptr() for p in self.parts], np.uint64))
        self.rep, ctl = zeros(fusion.taille_repertoire(E)), zeros(16)
        fz.monter_couche(vue(self.table), E, dims, vue(self.rep), vue(ctl))
        assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]
        r = np.stack([O.synth_normale_bf16(graine, 3, e, dims.colonnes[0], 0.02) for e in range(E)])
        self.r16 = dev((r.view(np.uint32) >> 16).astype(np.uint16))


def _pas(fz, couche, E, dims, k, N, x, residu0, sans_alloc):
    res, xd = dev(residu0), dev(x)
    idx, w, ctl = zeros(32), zeros(32), zeros(16)
    args = (vue(couche.rep), E, vue(couche.luts), dims, vue(couche.r16), None, vue(xd), k, vue(res), vue(idx),
            vue(w), vue(ctl))
    print(f"no-alloc test: E={E} k={k} dims={list(dims.lignes)}x{list(dims.colonnes)} N={N} "
          f"sans_alloc={sans_alloc}", flush=True)
    if sans_alloc:
        fz.couche_moe_sans_alloc(*args, *N)
    else:
        tr = zeros(fusion.taille_travail_couche(dims, E, k, N[1]))
        fz.couche_moe(*args, vue(tr), *N)
    return (hote(res, np.float32).copy(), hote(idx, np.uint32)[:k].copy(), hote(w, np.float32)[:k].copy(),
            hote(ctl, np.uint32).copy())


def test_allocation_free_step_equals_the_allocating_one():
    fz = fusion.Fusion()
    cas = [(2050, 16, DimsExpert.gpt_oss(), 4, (2, 16)),
           (2051, 6, DimsExpert.de([256, 256, 320], [320, 320, 256]), 2, (2, 8))]
    for graine, E, dims, k, N in cas:
        assert fusion.taille_travail_couche(dims, E, k, N[1]) <= fusion.octets_scratch()
        couche = Couche(fz, graine, E, dims, N)
        C_, D = dims.colonnes[0], dims.lignes[2]
        for t in range(2):
            x = O.synth_normale_bf16(graine, 4, t, C_, 1.0)
            residu0 = O.synth_normale_bf16(graine, 5, t, D, 0.5)
            a = _pas(fz, couche, E, dims, k, N, x, residu0, False)
            b = _pas(fz, couche, E, dims, k, N, x, residu0, True)
            assert list(a[3]) == [0, 0, 0, 0] and list(b[3]) == [0, 0, 0, 0]
            assert (a[1] == b[1]).all() and (a[2].view(np.uint32) == b[2].view(np.uint32)).all()
            assert (a[0].view(np.uint32) == b[0].view(np.uint32)).all(), (graine, t)
            assert np.abs(a[0] - residu0).max() > 0
        couche.c.liberer()


def test_step_larger_than_the_scratch_is_refused():
    fz = fusion.Fusion()
    dims, E, k, N = DimsExpert.gpt_oss(), 128, 8, (4, 16)
    assert fusion.taille_travail_couche(dims, E, k, N[1]) > fusion.octets_scratch()
    z = zeros(1 << 20)
    with pytest.raises(ErreurUsage, match="memoire statique"):
        fz.couche_moe_sans_alloc(vue(z), E, vue(z), dims, vue(z), None, vue(z), k, vue(z), vue(z), vue(z), vue(z),
                                 *N)
