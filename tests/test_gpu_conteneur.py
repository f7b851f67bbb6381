"""The GPU path fed from a .trc file, as the reference engine is fed (trc-ordo/src/lib.rs:389-420,
746-760): the file is opened and checked, the layer LUTs come from its TABLES, the parts are read
with their directory fingerprints checked, the router from RÉSIDENTS.

Full-size, size-independent checks: every expert of a gpt-oss-shape file is decoded on the GPU into
its SoA slot and the slot's empreinte64 must equal the directory's canonical fingerprint
(empreinte_emplacement, trc-ordo/src/lib.rs:238-262) — one flipped decoded bit anywhere in the 13 MB
slot fails. Then the fused MoE layer runs on parts and router read from the file and is compared
with the oracle chain, tolerance 1e-5 * max|y| (the reference's GEMV threshold).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import oracle_ffi as O  # noqa: E402
from gpu_outils import dev, hote, vue, zeros  # noqa: E402
from test_gpu_fusion import _mlp_oracle  # noqa: E402
from troncons_amd import codeur, fusion  # noqa: E402
from troncons_amd import conteneur as T  # noqa: E402
from troncons_amd import noyaux as K  # noqa: E402
from troncons_amd.noyaux import DimsExpert  # noqa: E402

GPT = DimsExpert.gpt_oss()
GRAINE, E, KK, N = 2029, 8, 4, (4, 16)
TOL = 1e-5


@pytest.fixture(scope="module")
def fichier(tmp_path_factory):
    assert torch.cuda.is_available()
    chemin = tmp_path_factory.mktemp("trc") / "gpt-oss-synth.trc"
    print(f"\nwriting {chemin} (1 layer x {E} experts, gpt-oss shape)", flush=True)
    T.synth_fichier(chemin, GRAINE, 1, E, KK, GPT, N_delta=N[0], N_codes=N[1], n_fils=16)
    return T.Fichier.ouvrir(chemin)


def _luts(f):
    fr = f.freqs_couche(0)
    luts = K.luts_couche([[fr[j][t] for t in range(4)] for j in range(3)])
    assert (luts == O.luts_couche(fr)).all()
    return luts


def test_decoded_slots_hash_to_the_directory(fichier):
    f = fichier
    nk = K.Noyaux()
    luts = dev(_luts(f))
    te = K.taille_emplacement(GPT)
    for x in range(E):
        print(f"expert {x}: read, decode, fingerprint", flush=True)
        en = f.entree(0, x)
        p = dev(f.lire_partie(0, x))
        slot, ctl = zeros(te), zeros(16)
        nk.decoder_expert(vue(p), vue(slot), vue(luts), GPT, vue(ctl))
        s = hote(slot)
        assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]
        assert T.empreinte_emplacement(s, GPT) == en.empreinte_canonique
        assert en.empreinte_canonique != en.empreinte_origine  # the generated experts do carry nibble 8


def test_fused_moe_layer_from_the_file(fichier):
    f = fichier
    fz = fusion.Fusion()
    luts = dev(_luts(f))
    parts = [dev(f.lire_partie(0, x)) for x in range(E)]
    table = dev(np.array([p.data_ptr() for p in parts], np.uint64))
    rep, ctl0 = zeros(fusion.taille_repertoire(E)), zeros(16)
    fz.monter_couche(vue(table), E, GPT, vue(rep), vue(ctl0))
    assert list(hote(ctl0, np.uint32)) == [0, 0, 0, 0]
    (r,) = [r for r in f.residents() if r.nom == "blk.0.ffn_gate_inp.weight"]
    assert (r.type_ggml, r.n_dims, r.ne[0], r.ne[1]) == (30, 2, 2880, E)
    r16 = f.donnees_resident(r).view(np.uint16).reshape(E, 2880)
    routeur = (r16.astype(np.uint32) << 16).view(np.float32)
    x = O.synth_normale_bf16(GRAINE, 4, 0, 2880, 1.0)
    residu0 = np.zeros(2880, np.float32)
    rd, xd, res = dev(r16), dev(x), dev(residu0)
    idx, w, ctl = zeros(32), zeros(32), zeros(16)
    tr = zeros(fusion.taille_travail_couche(GPT, E, KK, N[1]))
    fz.couche_moe(vue(rep), E, vue(luts), GPT, vue(rd), None, vue(xd), KK, vue(res), vue(idx), vue(w), vue(ctl),
                  vue(tr), *N)
    got = hote(res, np.float32)
    assert list(hote(ctl, np.uint32)) == [0, 0, 0, 0]
    oi, ow = O.routeur_topk(O.gemv_f32(routeur, x), KK)
    assert (hote(idx, np.uint32)[:KK] == oi).all()
    sorties, sorties64 = [], []
    for e in oi:
        bl, bi = codeur.synth_expert(GRAINE, 0, int(e), GPT)
        ex = type("E", (), {})()
        ex.attendu = np.concatenate([O.blocs_vers_soa(bl[j], 2880, 2880, bi[j], canonique=True) for j in range(3)])
        s, s64 = _mlp_oracle(ex, x, GPT)
        sorties.append(s)
        sorties64.append(s64)
    ref = O.combiner(residu0, np.concatenate(sorties), 2880, ow, KK, 2880)
    ref64 = sum(float(ow[i]) * sorties64[i] for i in range(KK))
    assert np.abs(got - ref).max() <= TOL * np.abs(ref).max()
    assert np.abs(got - ref64).max() <= TOL * np.abs(ref64).max()
