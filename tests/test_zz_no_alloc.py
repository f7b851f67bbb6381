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


def test_allocation_free_step_replays_from_a_graph():
    """The step captured into a HIP graph after the device's context is created (which resolves the
    scratch address): every replay, with eager copies and synchronisations between them, gives the
    allocating step's routing, weights and residual bits."""
    from troncons_amd import pilote
    fz = fusion.Fusion()
    graine, E, dims, k, N = 2052, 16, DimsExpert.gpt_oss(), 4, (1, 16)
    couche = Couche(fz, graine, E, dims, N)
    C_, D = dims.colonnes[0], dims.lignes[2]
    x = O.synth_normale_bf16(graine, 4, 0, C_, 1.0)
    residu0 = O.synth_normale_bf16(graine, 5, 0, D, 0.5)
    a = _pas(fz, couche, E, dims, k, N, x, residu0, False)
    assert list(a[3]) == [0, 0, 0, 0]
    ctx = pilote.Contexte(0)
    xd, r0, res = dev(x), dev(residu0), dev(residu0)
    idx, w, ctl = zeros(32), zeros(32), zeros(16)
    args = (vue(couche.rep), E, vue(couche.luts), dims, vue(couche.r16), None, vue(xd), k, vue(res), vue(idx),
            vue(w), vue(ctl))
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    print("no-alloc graph test: capturing the step", flush=True)
    with torch.cuda.graph(g, stream=s):
        fz.couche_moe_sans_alloc(*args, *N, f=s)
    for rep in range(3):
        res.copy_(r0)
        ctl.zero_()
        idx.zero_()
        torch.cuda.synchronize()
        print(f"no-alloc graph test: replay {rep}", flush=True)
        g.replay()
        torch.cuda.synchronize()
        assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0], rep
        assert (hote(idx, np.uint32)[:k] == a[1]).all(), rep
        assert (hote(w, np.float32)[:k].view(np.uint32) == a[2].view(np.uint32)).all(), rep
        assert (hote(res, np.float32).view(np.uint32) == a[0].view(np.uint32)).all(), rep
    del g
    ctx.detruire()
    couche.c.liberer()


def test_step_larger_than_the_scratch_is_refused():
    fz = fusion.Fusion()
    dims, E, k, N = DimsExpert.gpt_oss(), 128, 8, (4, 16)
    assert fusion.taille_travail_couche(dims, E, k, N[1]) > fusion.octets_scratch()
    z = zeros(1 << 20)
    with pytest.raises(ErreurUsage, match="memoire statique"):
        fz.couche_moe_sans_alloc(vue(z), E, vue(z), dims, vue(z), None, vue(z), k, vue(z), vue(z), vue(z), vue(z),
                                 *N)
