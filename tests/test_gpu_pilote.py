"""The driver half of the C-ABI on the GPU, used alone (this module never touches torch: every
launch gets an explicit stream of the driver half): a context, two
streams, events, device memory, pinned and mapped host memory, asynchronous copies and fills, and
the Noyaux entry points launched on those streams — the way the reference engine drives its kernels
through trc_cuda (moteur/crates/trc-cuda/src/lib.rs:160-623) and its scheduler reads the router
through a mapped mailbox (trc-ordo/src/lib.rs:1054-1116, passe.cuh:447-514).

- Router to mailbox: routeur_topk writes the k indices and weights into mapped host memory, then the
  sequence word; the host polls that word without synchronizing the stream, then reads the choice,
  which must equal the oracle's routeur_topk (ties by index).
- Copy -> decode -> GEMV across two streams: a part copied from pinned memory on a copy stream, an
  event recorded there, the compute stream waiting for it, the reference decoder writing the slot,
  the reference GEMV over it (bit-exact against the oracle), results copied back to pinned memory,
  timed events on both streams.
"""
from __future__ import annotations

import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import oracle_ffi as O  # noqa: E402
from troncons_amd import codeur  # noqa: E402
from troncons_amd import noyaux as K  # noqa: E402
from troncons_amd import pilote as P  # noqa: E402
from troncons_amd.noyaux import DimsExpert  # noqa: E402


@pytest.fixture(scope="module")
def ctx():
    c = P.Contexte(0)
    yield c
    c.detruire()


def test_context_and_attributes(ctx):
    assert ctx.nom() != ""
    libre, totale = ctx.memoire()
    assert 0 < libre <= totale
    assert ctx.attribut(P.UNITES_DE_CALCUL) > 0
    assert ctx.attribut(P.PROJECTION_HOTE) == 1
    assert ctx.attribut(P.LDS_PAR_BLOC) >= 65536
    assert ctx.attente_effective() in (P.ATTENTE_AUTO, P.ATTENTE_ACTIVE, P.ATTENTE_CEDE, P.ATTENTE_BLOQUANTE)
    a, b = P.Flux(ctx, priorite_haute=True), P.Flux(ctx)
    assert a.priorite() == b.priorite()  # every stream at the default priority
    assert a.fini() and b.fini()
    a.detruire()
    b.detruire()


def test_router_to_mapped_mailbox(ctx):
    E, k, seq = 128, 4, 7
    rng = np.random.default_rng(5)
    logits = rng.standard_normal(E).astype(np.float32)
    logits[[9, 40]] = logits.max() + 1.0  # a tie at the top: the smaller index first
    logits[77] = np.float32(np.nan)
    calcul = P.Flux(ctx)
    hl = P.HoteEpingle(ctx, 4 * E)
    hl.tranche()[:4 * E] = logits.view(np.uint8)
    dl, idx, w = P.MemoireCarte(ctx, 4 * E), P.MemoireCarte(ctx, 32), P.MemoireCarte(ctx, 32)
    boite = P.HoteEpingle(ctx, 4096, projetee=True)
    boite.tranche()[:] = 0
    assert boite.adresse_carte() is not None
    P.copier_vers_carte(dl.tout(), hl, 0, 4 * E, calcul)
    K.Noyaux().routeur_topk(dl.tout(), E, k, idx.tout(), w.tout(), boite=boite.adresse_carte(), sequence=seq,
                            f=calcul)
    t0 = time.time()
    while boite.lire_volatil_u32(0) != seq:  # the sequence word is written last
        assert time.time() - t0 < 10.0, "mailbox never written"
    mots = np.array([boite.lire_volatil_u32(4 * i) for i in range(1 + 2 * k)], np.uint32)
    oi, ow = O.routeur_topk(logits, k)
    assert list(mots[1:1 + k]) == list(oi) and oi[0] == 9 and oi[1] == 40
    assert np.abs(mots[1 + k:].view(np.float32) - ow).max() <= 1e-6
    calcul.synchroniser()
    for m in (hl, boite):
        m.liberer()
    for m in (dl, idx, w):
        m.liberer()
    calcul.detruire()


def test_copy_decode_gemv_on_two_streams(ctx):
    dims = DimsExpert.de([256, 256, 320], [512, 512, 256])
    bl, bi = codeur.synth_expert(2026, 0, 3, dims)
    freqs = [codeur.tables([bl[j]], dims.lignes[j], dims.colonnes[j] // 32) for j in range(3)]
    partie, _ = codeur.partie(bl, bi, freqs, dims, N_delta=8, N_codes=16)
    luts = O.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)])
    R, C_ = dims.lignes[2], dims.colonnes[2]
    x = O.synth_normale_bf16(2026, 1, 3, C_, 1.0)
    nk = K.Noyaux()
    calcul, copie = P.Flux(ctx), P.Flux(ctx)
    ev_copie = P.Evenement(ctx)
    debut, fin = P.Evenement(ctx, horodate=True), P.Evenement(ctx, horodate=True, bloquant=True)
    hp = P.HoteEpingle(ctx, len(partie) + luts.nbytes + x.nbytes)
    t = hp.tranche()
    t[:len(partie)] = np.frombuffer(partie, np.uint8)
    t[len(partie):len(partie) + luts.nbytes] = luts.view(np.uint8)
    t[len(partie) + luts.nbytes:len(partie) + luts.nbytes + x.nbytes] = x.view(np.uint8)
    dp, dl, dx = P.MemoireCarte(ctx, len(partie)), P.MemoireCarte(ctx, luts.nbytes), P.MemoireCarte(ctx, x.nbytes)
    emplacement = P.MemoireCarte(ctx, K.taille_emplacement(dims))
    ctl, y = P.MemoireCarte(ctx, 16), P.MemoireCarte(ctx, 4 * R)
    debut.enregistrer(copie)
    P.copier_vers_carte(dp.tout(), hp, 0, len(partie), copie)
    ev_copie.enregistrer(copie)
    P.copier_vers_carte(dl.tout(), hp, len(partie), luts.nbytes, calcul)
    P.copier_vers_carte(dx.tout(), hp, len(partie) + luts.nbytes, x.nbytes, calcul)
    ctl.remplir(ctl.tout(), 0, calcul)
    y.remplir(y.tout(), 0xFF, calcul)
    calcul.attendre(ev_copie)  # the decode waits for the part's copy on the other stream
    nk.decoder_expert(dp.tout(), emplacement.tout(), dl.tout(), dims, ctl.tout(), f=calcul)
    d2 = K.disposition(dims, 2)
    nk.gemv(emplacement.vue(d2.base, d2.pas), dx.tout(), y.tout(), R, C_, f=calcul)
    retour = P.HoteEpingle(ctx, 4 * R + 16)
    P.copier_vers_hote(retour, 0, y.tout(), calcul)
    P.copier_vers_hote(retour, 4 * R, ctl.tout(), calcul)
    fin.enregistrer(calcul)
    fin.attendre()
    assert fin.fini() and calcul.fini() and copie.fini()
    assert fin.ms_depuis(debut) >= 0.0
    r = retour.tranche()
    assert (r[4 * R:4 * R + 16].view(np.uint32) == 0).all(), "control words"
    slot = O.blocs_vers_soa(bl[2], R, C_, bi[2], canonique=True)
    attendu = O.gemv_mxfp4(slot, x, R, C_)
    assert (r[:4 * R].view(np.uint32) == attendu.view(np.uint32)).all()
    # a device-to-device copy and a fill of part of a view
    y2 = P.MemoireCarte(ctx, 4 * R)
    P.copier_carte_carte(y2.tout(), y.tout(), calcul)
    y2.remplir(y2.vue(4, 8), 0x00, calcul)
    P.copier_vers_hote(retour, 0, y2.tout(), calcul)
    calcul.synchroniser()
    r2 = retour.tranche()[:4 * R].view(np.uint32)
    assert r2[1] == 0 and r2[2] == 0 and (np.delete(r2, [1, 2]) == np.delete(attendu.view(np.uint32), [1, 2])).all()
    with pytest.raises(K.ErreurUsage):
        P.copier_carte_carte(y.vue(0, 4), y2.tout(), calcul)
    for m in (hp, retour):
        m.liberer()
    for m in (dp, dl, dx, emplacement, ctl, y, y2):
        m.liberer()
    for e in (ev_copie, debut, fin):
        e.detruire()
    calcul.detruire()
    copie.detruire()
