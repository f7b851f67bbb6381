"""A decode step through whole layers (troncons_amd/modele.py, the reference's Modele, trc-modele
src/lib.rs:476-568) on the GPU, against the oracle chain run the same way on the CPU: embedding,
per layer RMSNorm, Q/K/V Q8_0 GEMVs, YaRN, f16 KV write, sink attention (a sliding-window layer
whose ring wraps, and a full-cache layer), output projection and residual, post-norm, router top-k,
the k experts decoded from their .trc parts (the oracle's decoder and GEMV in the reference order),
SwiGLU and the ordered combine; then the output norm, Q8_0 logits and argmax.

The same step issued by the native driver (csrc/modele.cpp, one call per token) gives the Python
driver's logits bit for bit. Teacher forcing (a fixed token sequence) keeps both chains on the same
inputs. Per step: the
router's choices equal the oracle's in every layer, the logits are within 1e-4 * max|z| of the
oracle's (each layer's experts meet 1e-5; attention and the projections follow the reference order),
and the greedy token is the oracle's wherever its margin over the runner-up exceeds that tolerance.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle_ffi as O  # noqa: E402
from troncons_amd import modele as Mo  # noqa: E402
from troncons_amd.noyaux import DimsExpert, ParamsRope  # noqa: E402


def _hyper(**k):
    v = dict(couches=2, d=256, tetes=8, tetes_kv=2, experts=8, actifs=4, vocab=1000, eps=1e-5,
             rope=ParamsRope.gpt_oss(), fenetre=8, contexte=32, dims=DimsExpert.de([256] * 3, [256] * 3),
             n_delta=4, n_codes=8)
    v.update(k)
    return Mo.Hyper(**v)


class ChaineOracle:
    """The same step on the CPU with the oracle's functions."""

    def __init__(self, h, couches, emb, norme, sortie):
        self.h, self.couches, self.emb, self.norme, self.sortie = h, couches, emb, norme, sortie
        self.ck = [np.zeros((h.anneau(l) or h.contexte) * h.dkv, np.uint16) for l in range(h.couches)]
        self.cv = [c.copy() for c in self.ck]
        self.luts = [O.luts_couche([[p.freqs[j][t] for t in range(4)] for j in range(3)]) for p in couches]
        self.routeurs = [(p.routeur.astype(np.uint32) << 16).view(np.float32).reshape(h.experts, h.d) for p in couches]
        self._slots = {}

    def slot(self, l, e):
        if (l, e) not in self._slots:
            lg, cl = list(self.h.dims.lignes), list(self.h.dims.colonnes)
            s, ctl = O.decoder_expert(self.couches[l].parties[e].tobytes(), self.luts[l], lg, cl)
            assert (ctl == 0).all()
            self._slots[(l, e)] = s
        return self._slots[(l, e)]

    def mlp(self, l, e, x):
        lg, cl = list(self.h.dims.lignes), list(self.h.dims.colonnes)
        d = [O.disposition_j(lg, cl, j) for j in range(3)]
        s = self.slot(l, e)
        g = O.gemv_mxfp4(s[d[0].base:d[0].base + d[0].pas], x, lg[0], cl[0])
        u = O.gemv_mxfp4(s[d[1].base:d[1].base + d[1].pas], x, lg[1], cl[1])
        return O.gemv_mxfp4(s[d[2].base:d[2].base + d[2].pas], O.swiglu_oai(g, u), lg[2], cl[2])

    def pas(self, jeton, pos):
        h = self.h
        d, dq, dkv = h.d, h.dq, h.dkv
        x = O.ligne_q8_0(self.emb, jeton, d)
        choix = []
        for l, p in enumerate(self.couches):
            hh = O.rmsnorm(x, p.attn_norm, d, 1, h.eps)
            q = O.gemv_q8_0(p.wq, hh, p.bq, dq, d)
            k = O.gemv_q8_0(p.wk, hh, p.bk, dkv, d)
            v = O.gemv_q8_0(p.wv, hh, p.bv, dkv, d)
            q, k = O.rope_yarn(q, k, h.tetes, h.tetes_kv, pos, O.rope_gpt_oss())
            an = h.anneau(l)
            self.ck[l], self.cv[l] = O.ecrire_kv(k, v, self.ck[l], self.cv[l], dkv, pos % an if an else pos)
            fin = pos + 1
            pa = O.ParamsAttention(h.tetes, h.tetes_kv, 64, max(fin - an, 0) if an else 0, fin, an, 0.125, 0)
            a = O.attention(q, self.ck[l], self.cv[l], p.puits, pa)
            o = O.gemv_q8_0(p.wo, a, p.bo, d, dq)
            x = O.combiner(x, o, d, None, 1, d)
            h2 = O.rmsnorm(x, p.post_norm, d, 1, h.eps)
            oi, ow = O.routeur_topk(O.gemv_f32(self.routeurs[l], h2, p.routeur_biais), h.actifs)
            choix.append(oi)
            x = O.combiner(x, np.concatenate([self.mlp(l, int(e), h2) for e in oi]), d, ow, h.actifs, d)
        z = O.gemv_q8_0(self.sortie, O.rmsnorm(x, self.norme, d, 1, h.eps), None, h.vocab, d)
        return z, choix


@pytest.mark.parametrize("graine", [2040, 2041])
def test_decode_steps_equal_the_oracle_chain(graine):
    assert torch.cuda.is_available()
    h = _hyper()
    couches, emb, norme, sortie = Mo.poids_synthetiques(h, graine)
    m = Mo.Modele(h, couches, emb, norme, sortie)
    mn = Mo.Modele(h, couches, emb, norme, sortie)  # the same step issued by the native driver
    ref = ChaineOracle(h, couches, emb, norme, sortie)
    jetons = np.random.default_rng(graine).integers(0, h.vocab, 14)
    choix_gpu = []
    for pos, tok in enumerate(jetons):
        print(f"seed {graine} position {pos}", flush=True)
        z_ref, choix = ref.pas(int(tok), pos)
        choix_gpu = []
        m.enchasser(int(tok))
        for l in range(h.couches):
            m.debut_couche(l, pos)
            m.fin_couche(l)
            choix_gpu.append(m.indices())
        m.sortie()
        z = m.logits()
        mn.pas_natif(int(tok), pos)
        assert (mn.logits_natif().view(np.uint32) == z.view(np.uint32)).all(), pos
        assert mn.jeton_natif() == m.jeton()
        for l in range(h.couches):
            assert (choix_gpu[l] == choix[l]).all(), (pos, l, choix_gpu[l], choix[l])
        assert np.abs(z - z_ref).max() <= 1e-4 * np.abs(z_ref).max(), pos
        deux = np.sort(z_ref)[-2:]
        if deux[1] - deux[0] > 1e-4 * np.abs(z_ref).max():
            assert m.jeton() == int(np.argmax(z_ref)), pos
    assert (m.controles() == 0).all() and (mn.controles_natif() == 0).all()


def test_decode_step_head_from_32768_rows():
    """A vocabulary of 33001 rows takes the head through the four-rows-per-half-wavefront GEMV: the
    logits equal the oracle's Q8_0 GEMV of the normed row the step left in hh, bit for bit, and the
    native driver's logits equal the Python driver's."""
    from gpu_outils import hote
    h = _hyper(vocab=33001, couches=1)
    couches, emb, norme, sortie = Mo.poids_synthetiques(h, 2042)
    m = Mo.Modele(h, couches, emb, norme, sortie)
    mn = Mo.Modele(h, couches, emb, norme, sortie)
    for pos, tok in enumerate([7, 33000, 12345]):
        print(f"position {pos}", flush=True)
        m.pas(tok, pos)
        z = m.logits()
        hh = hote(m.hh, np.float32)
        assert (O.gemv_q8_0(sortie, hh, None, h.vocab, h.d).view(np.uint32) == z.view(np.uint32)).all(), pos
        mn.pas_natif(tok, pos)
        assert (mn.logits_natif().view(np.uint32) == z.view(np.uint32)).all(), pos
        assert mn.jeton_natif() == m.jeton()


def test_model_refuses_position_past_context():
    from troncons_amd.noyaux import ErreurUsage
    h = _hyper(couches=1, contexte=4)
    couches, emb, norme, sortie = Mo.poids_synthetiques(h, 7)
    m = Mo.Modele(h, couches, emb, norme, sortie)
    with pytest.raises(ErreurUsage):
        m.debut_couche(0, 4)
    with pytest.raises(ErreurUsage):
        m.pas_natif(0, 4)
    with pytest.raises(ErreurUsage):
        m.pas_natif(h.vocab, 0)
