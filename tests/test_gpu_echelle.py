"""GPU parity at the workloads' real sizes, through the C-ABI.

- Config 3: the fused MoE layer over 128 resident gpt-oss-120b experts in the bench's encoding
  (gate and up: CODES_CTX tiles of 32 macro-steps, DELTA tiles of 2; down: 16 and 1; each tile's
  DELTA decoded inside the CODES kernels), 20 seeded tokens, some with tied router rows and some
  with NaN rows. Indices
  must equal the oracle's routeur_topk on the oracle's router logits (reference gemv_f32 order),
  weights within 1e-6, and the residual within 1e-5 * max|change| of the f64 MLP chain computed from
  the uncompressed weights (and, for the first tokens, of the reference's own f32 chain).
- Config 5: the bench's 512-position prefill with Zipf(1.1) routing over the same 128 experts; every
  position of the most-chosen expert and 24 other seeded positions checked against the f64 chain.
- Config 4: one token through 36 resident layers x 128 experts (parts copied per layer from the
  128-expert pool, permuted per layer, each layer with its own router, about 52 GB resident), each
  layer's routing and residual change checked against the oracle; the streaming variant (parts in
  pinned host memory, router top-k read by the host, the chosen parts copied on a side stream and
  decoded as they land) must give the resident run's bits at every layer.

Tolerance: 1e-5 * max|change| (the reference's GEMV threshold, decisions/ARCHITECTURE.md §5.6);
routing exact; router weights 1e-6 (f64 softmax rounded once on both sides).
"""
from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle_ffi as O  # noqa: E402
from gpu_outils import DEV, carte_parallele, dev, hote, mlp_f64, vue, zeros  # noqa: E402
from troncons_amd import codeur, fusion  # noqa: E402
from troncons_amd import noyaux as K  # noqa: E402
from troncons_amd.noyaux import DimsExpert, VueCarte  # noqa: E402

GPT = DimsExpert.gpt_oss()
C_ = 2880
E, KTOP = 128, 4
N_MATRICES = ((2, 2, 1), (32, 32, 16))  # (N_delta, N_codes) per matrix (gate, up, down): the bench's
N = (1, 16)  # what the API calls take: the down matrix's, which size the workspace and choose the plan
GRAINE = 2040
TOL = 1e-5


def _r16(routeur_f32: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(routeur_f32).view(np.uint32) >> 16).astype(np.uint16)


class Pool:
    """The 128-expert layer, encoded once: parts in one device allocation (each 256-aligned), the
    address table, the mounted directory, the LUTs, and the parts in host memory."""

    def __init__(self, fz):
        self.c = codeur.CoucheSynthetique(GRAINE, 0, E, GPT, N_delta=N_MATRICES[0], N_codes=N_MATRICES[1])
        self.parts = [self.c.partie(e) for e in range(E)]
        tailles = np.array([p.size for p in self.parts], np.int64)
        self.tailles = tailles
        self.decal = np.concatenate([[0], np.cumsum((tailles + 255) // 256 * 256)[:-1]]).astype(np.int64)
        self.octets = int(self.decal[-1] + tailles[-1])
        self.hote = np.zeros(self.octets, np.uint8)
        for e in range(E):
            self.hote[self.decal[e]:self.decal[e] + tailles[e]] = self.parts[e]
        self.bloc = dev(self.hote)
        freqs = self.c.freqs()
        self.luts_np = O.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)])
        self.luts = dev(self.luts_np)
        self.fz = fz

    def monter(self, bloc: torch.Tensor, perm: np.ndarray):
        """Directory of a layer whose expert e is pool part perm[e], in the copy `bloc`."""
        table = dev(np.array([bloc.data_ptr() + int(self.decal[p]) for p in perm], np.uint64))
        rep, ctl = zeros(fusion.taille_repertoire(E)), zeros(16)
        self.fz.monter_couche(vue(table), E, GPT, vue(rep), vue(ctl))
        assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]
        return rep, table


@pytest.fixture(scope="module")
def fz():
    assert torch.cuda.is_available()
    return fusion.Fusion()


@pytest.fixture(scope="module")
def pool(fz):
    p = Pool(fz)
    yield p
    p.c.liberer()
    torch.cuda.empty_cache()


_blocs_cache: dict = {}


def _blocs(e: int):
    if e not in _blocs_cache:
        _blocs_cache[e] = codeur.synth_expert(GRAINE, 0, int(e), GPT)
    return _blocs_cache[e]


def _sorties_f64(besoins: dict) -> dict:
    """{expert: X (C x n)} -> {expert: f64 MLP outputs (D x n)}, experts in parallel."""
    experts = sorted(besoins)

    def un(e):
        bl, bi = _blocs(e)
        return mlp_f64(bl, bi, besoins[e])
    return dict(zip(experts, carte_parallele(un, experts)))


def _routeur_jeton(base: np.ndarray, x: np.ndarray, t: int) -> np.ndarray:
    """The router of token t: tokens 3-5 have two tied pairs of rows turned towards x (so the ties
    sit in the top-4), tokens 6-8 one NaN row among tied winners, token 9 two NaN rows and a tie."""
    r = base.copy()
    rng = np.random.default_rng(GRAINE + 1000 + t)
    a, b, c, d, n1, n2 = (int(v) for v in rng.choice(E, size=6, replace=False))
    m = float(np.abs(base.astype(np.float64) @ x).max())

    def gagnant(i, marge=4.0):
        # a power-of-two scale (the row stays bf16-exact) that lifts the row's logit above every
        # other row's by `marge`
        v = float(base[i].astype(np.float64) @ x)
        s = 2.0 ** np.ceil(np.log2(marge * m / max(abs(v), 1e-30)))
        return (base[i] * np.float32(s if v > 0 else -s)).astype(np.float32)
    if 3 <= t <= 5:
        r[a] = r[b] = gagnant(a, 64.0)
        r[c] = r[d] = gagnant(c)
    elif 6 <= t <= 8:
        r[a] = r[b] = gagnant(a)
        r[n1] = np.float32(np.nan)
        r[c] = gagnant(c)
    elif t == 9:
        r[a] = r[b] = gagnant(a)
        r[n1] = np.float32(np.nan)
        r[n2] = np.float32(np.nan)
    return r


def test_moe_layer_128_experts(fz, pool):
    """Config 3 at its size: 20 tokens through the fused layer over the 128 resident experts."""
    T = 20
    rep, _table = pool.monter(pool.bloc, np.arange(E))
    base = np.stack([O.synth_normale_bf16(GRAINE, 3, e, C_, 0.02) for e in range(E)])
    tr = zeros(fusion.taille_travail_couche(GPT, E, KTOP, N[1]))
    res_gpu, idx_gpu, w_gpu, routes, x_tok, r0 = [], [], [], [], [], []
    for t in range(T):
        x = O.synth_normale_bf16(GRAINE, 4, t, C_, 1.0)
        residu0 = O.synth_normale_bf16(GRAINE, 5, t, C_, 0.5)
        routeur = _routeur_jeton(base, x, t)
        xd, res, rd = dev(x), dev(residu0), dev(_r16(routeur))
        idx, w, ctl = zeros(32), zeros(32), zeros(16)
        print(f"config3 token {t}: 128 experts, k=4, N={N_MATRICES}", flush=True)
        fz.couche_moe(vue(rep), E, vue(pool.luts), GPT, vue(rd), None, vue(xd), KTOP, vue(res), vue(idx), vue(w),
                      vue(ctl), vue(tr), *N)
        assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0], t
        res_gpu.append(hote(res, np.float32).copy())
        idx_gpu.append(hote(idx, np.uint32)[:KTOP].copy())
        w_gpu.append(hote(w, np.float32)[:KTOP].copy())
        routes.append(routeur)
        x_tok.append(x)
        r0.append(residu0)
    # routing: the oracle's top-k on the oracle's logits
    choix = []
    for t in range(T):
        logits = O.gemv_f32(routes[t], x_tok[t])
        oi, ow = O.routeur_topk(logits, KTOP)
        if 3 <= t <= 5:  # two tied pairs fill the top-4: the index order decides within each pair
            assert len(set(float(logits[int(i)]) for i in oi)) == 2, t
        if 6 <= t <= 9:
            assert np.isnan(logits).any() and not any(np.isnan(logits[int(i)]) for i in oi)
        assert (idx_gpu[t] == oi).all(), (t, idx_gpu[t], oi)
        assert np.abs(w_gpu[t] - ow).max() <= 1e-6, t
        choix.append((oi, ow))
    # residual: f64 chain from the uncompressed weights, experts computed once over all their tokens
    besoins: dict = {}
    for t, (oi, _) in enumerate(choix):
        for e in oi:
            besoins.setdefault(int(e), []).append(t)
    sorties = _sorties_f64({e: np.stack([x_tok[t] for t in ts], 1).astype(np.float64) for e, ts in besoins.items()})
    for t, (oi, ow) in enumerate(choix):
        ref = r0[t].astype(np.float64)
        for q, e in enumerate(oi):
            ref = ref + float(ow[q]) * sorties[int(e)][:, besoins[int(e)].index(t)]
        d = np.abs(ref - r0[t]).max()
        assert np.abs(res_gpu[t] - ref).max() <= TOL * d, (t, np.abs(res_gpu[t] - ref).max() / d)
    # the reference's own f32 chain for the first tokens (gemv_mxfp4 order, swiglu_oai, combiner)

    def chaine32(arg):
        e, x = arg
        bl, bi = _blocs(e)
        sl = [O.blocs_vers_soa(bl[j], C_, C_, bi[j], canonique=True) for j in range(3)]
        g = O.gemv_mxfp4(sl[0], x, C_, C_)
        u = O.gemv_mxfp4(sl[1], x, C_, C_)
        return O.gemv_mxfp4(sl[2], O.swiglu_oai(g, u), C_, C_)
    for t in range(4):
        oi, ow = choix[t]
        s = carte_parallele(chaine32, [(int(e), x_tok[t]) for e in oi])
        ref32 = O.combiner(r0[t], np.concatenate(s), C_, ow, KTOP, C_)
        dd = np.abs(ref32 - r0[t]).max()
        assert np.abs(res_gpu[t] - ref32).max() <= TOL * dd, t


def test_prefill_512_positions_zipf(fz, pool):
    """Config 5 at its size: the bench's 512-position batch, Zipf(1.1) routing over 128 experts."""
    T = 512
    rep, _table = pool.monter(pool.bloc, np.arange(E))
    idx, w = codeur.routage_zipf(GRAINE + 5, T, E, KTOP)
    x = np.stack([O.synth_normale_bf16(GRAINE, 6, i, C_, 1.0) for i in range(T)])
    residu0 = np.stack([O.synth_normale_bf16(GRAINE, 8, i, C_, 0.25) for i in range(T)])
    xd, idd, wd, res = dev(x), dev(idx), dev(w), dev(residu0)
    ctl = zeros(16)
    tr = zeros(fusion.taille_travail_prefill(GPT, E, T, KTOP, N[1]))
    comptes = np.bincount(idx.reshape(-1), minlength=E)
    print(f"config5: {T} positions, Zipf 1.1 over {E} experts, most-chosen expert {int(comptes.argmax())} "
          f"with {int(comptes.max())} positions", flush=True)
    fz.prefill_moe(vue(rep), E, vue(pool.luts), GPT, vue(xd), T, vue(idd), vue(wd), KTOP, vue(res), vue(ctl),
                   vue(tr), *N)
    got = hote(res, np.float32).reshape(T, C_)
    assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]
    haut = int(comptes.argmax())
    positions = set(np.nonzero((idx == haut).any(1))[0].tolist())
    positions |= set(np.random.default_rng(GRAINE + 9).choice(T, size=24, replace=False).tolist())
    positions = sorted(positions)
    besoins: dict = {}
    for i in positions:
        for e in idx[i]:
            besoins.setdefault(int(e), []).append(i)
    sorties = _sorties_f64({e: x[ps].T.astype(np.float64) for e, ps in besoins.items()})
    for i in positions:
        ref = residu0[i].astype(np.float64)
        for q in range(KTOP):
            e = int(idx[i, q])
            ref = ref + float(w[i, q]) * sorties[e][:, besoins[e].index(i)]
        d = np.abs(ref - residu0[i]).max()
        assert np.abs(got[i] - ref).max() <= TOL * d, (i, np.abs(got[i] - ref).max() / d)


def test_36_layers_resident_and_streamed(fz, pool):
    """Config 4 at its size: a token through 36 resident layers x 128 experts, then the same token
    with the parts in pinned host memory, streamed per layer; bit-identical residuals."""
    L = 36
    perms = [np.random.default_rng(GRAINE + 200 + l).permutation(E) for l in range(L)]
    routeurs = [np.stack([O.synth_normale_bf16(GRAINE + 300 + l, 3, e, C_, 0.02) for e in range(E)])
                for l in range(L)]
    x = O.synth_normale_bf16(GRAINE, 7, 0, C_, 1.0)
    blocs = []
    for l in range(L):  # every layer holds its own copy of the parts: L x 1.45 GB resident
        b = torch.empty(pool.octets + 256, dtype=torch.uint8, device=DEV)
        v = b[(-b.data_ptr()) % 256:][:pool.octets]
        v.copy_(pool.bloc)
        v._garde = b
        blocs.append(v)
    print(f"config4: {L} layers x {E} experts resident ({L * pool.octets / 1e9:.1f} GB)", flush=True)
    couches = [pool.monter(blocs[l], perms[l]) for l in range(L)]
    luts = [dev(pool.luts_np) for _ in range(L)]
    r16 = [dev(_r16(r)) for r in routeurs]
    xd = dev(x)
    res = zeros(4 * C_)
    tr = zeros(fusion.taille_travail_couche(GPT, E, KTOP, N[1]))
    par_couche = []
    for l in range(L):
        idx, w, ctl = zeros(32), zeros(32), zeros(16)
        fz.couche_moe(vue(couches[l][0]), E, vue(luts[l]), GPT, vue(r16[l]), None, vue(xd), KTOP, vue(res), vue(idx),
                      vue(w), vue(ctl), vue(tr), *N)
        assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0], l
        par_couche.append((hote(idx, np.uint32)[:KTOP].copy(), hote(w, np.float32)[:KTOP].copy(),
                           hote(res, np.float32).copy()))
    print("config4: resident run done, checking every layer against the oracle", flush=True)
    choix = []
    for l in range(L):
        oi, ow = O.routeur_topk(O.gemv_f32(routeurs[l], x), KTOP)
        assert (par_couche[l][0] == oi).all(), (l, par_couche[l][0], oi)
        assert np.abs(par_couche[l][1] - ow).max() <= 1e-6, l
        choix.append((oi, ow))
    # every layer applies pool experts to the same x: one f64 MLP per distinct pool part
    utilises = sorted({int(perms[l][e]) for l in range(L) for e in choix[l][0]})
    sorties = _sorties_f64({p: x[:, None].astype(np.float64) for p in utilises})
    avant = np.zeros(C_, np.float32)
    for l in range(L):
        oi, ow = choix[l]
        delta = sum(float(ow[q]) * sorties[int(perms[l][e])][:, 0] for q, e in enumerate(oi))
        apres = par_couche[l][2]
        assert np.abs((apres.astype(np.float64) - avant) - delta).max() <= TOL * np.abs(delta).max(), l
        avant = apres
    del blocs, couches
    torch.cuda.empty_cache()

    # streaming variant through the native engine (trc_diffusion_*): the pool in pinned host memory;
    # per layer the router (gemv_f32 over the widened bf16 rows, then routeur_topk into the mapped
    # mailbox) on the compute stream, one host wait, the chosen parts copied on the engine's copy
    # stream, each expert run by trc_expert_fusionne once its copy has landed, then the combine
    from troncons_amd.diffusion import Diffusion
    epingle = torch.from_numpy(pool.hote).pin_memory()
    r32 = [dev(((r16_h.astype(np.uint32) << 16).view(np.float32))) for r16_h in (_r16(r) for r in routeurs)]
    calcul = torch.cuda.current_stream()
    couches_h = [(epingle, pool.decal[perms[l]], pool.tailles[perms[l]], vue(luts[l]), vue(r32[l])) for l in range(L)]
    moteur = Diffusion(couches_h, E, KTOP, GPT, *N)
    res2 = zeros(4 * C_)
    for l in range(L):
        sel = moteur.couche(l, vue(xd), vue(res2), f=calcul)
        assert (sel.astype(np.int64) == par_couche[l][0]).all(), l
        torch.cuda.synchronize()
        got = hote(res2, np.float32)
        assert (got.view(np.uint32) == par_couche[l][2].view(np.uint32)).all(), \
            (l, np.abs(got - par_couche[l][2]).max())
    assert list(moteur.controle()) == [0, 0, 0, 0]
    st = moteur.stats()
    assert st["couches"] == L and st["octets_copies"] == sum(
        int(pool.tailles[perms[l][e]]) for l in range(L) for e in par_couche[l][0])
    moteur.detruire()
    print("config4: streamed run equals the resident run at every layer", flush=True)
