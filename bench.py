#!/usr/bin/env python3
"""Benchmark of the fused expert path on one MI355X.

Default: 128 rANS-coded experts of gpt-oss-120b shape (.trc v1.2 level-0 parts,
seeded synthetic MXFP4) sit resident in HBM with a bf16 2880 x 128 router. A step is one token
through the MoE layer: router logits, top-4 with softmax weights, the 4 selected experts decoded
inside their fused GEMVs (gate/up -> SwiGLU -> down), and the weighted combine; the token sweep
uses 1000 seeded activations, so routing is uniform-random over the 1.45 GB layer. Prints ONE JSON
line: metric, value, unit, timing, config, the roofline of the dominant kernel and the CPU baseline.

Other measurement modes (not the driver's line): --config 1 (one down_proj matrix), --config 2 (one
expert MLP), both rotating over the 128 experts; --config 4 (a token through L resident MoE layers,
default 36, about 52 GB of parts; --ordo streams them from a .trc file through the native scheduler,
with --prechargement / --biais-cache); --config 5 (a batched prefill of 512 positions with Zipf
routing, grouped GEMM on the bf16 MFMA); --config 6 (a whole decode step: embedding,
L gpt-oss layers of Q8_0 attention and fused compressed MoE, the 201088-row head, argmax); --noyaux
(the reference kernel API over decoded VRAM slots: batched MXFP4 GEMVs of a layer step).
"""
from __future__ import annotations

import argparse
import json
import os
import pathlib
import struct
import sys
import time

RACINE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(RACINE))

METRIQUE = "MoE layer us/token @batch1 top-4; compressed-weight HBM GB/s (% of peak)"
PIC_HBM = 8000.0  # GB/s, MI355X
PART_CPU_PAR_GPU = 16  # host CPUs a one-GPU box grants this process
C_GPT = 2880


FICHIER_PMC = RACINE / "profiles" / "moe_config3_pmc.md"
FICHIER_PMC_PREFILL = RACINE / "profiles" / "prefill_config5_pmc.md"


def trafic_mesure(fichier=FICHIER_PMC):
    """HBM bytes per launch of the bench's dominant kernel (config 3: mean of the gate/up and down
    CODES launches; config 5: the slot decoder) from the committed counter summary (two rocprofv3
    --pmc runs, FETCH_SIZE then WRITE_SIZE, scaled by a copy kernel), or None."""
    try:
        for ligne in fichier.read_text().splitlines():
            if ligne.startswith("traffic_per_launch_bytes"):
                return int(ligne.split("=")[1])
    except (OSError, ValueError):
        pass
    return None


def lire_flux(partie: bytes):
    """{(kind, matrix): (offset, length)} from a part's stream table (ARCHITECTURE.md §4.8)."""
    n = struct.unpack_from("<H", partie, 10)[0]
    out = {}
    for i in range(n):
        e = 64 + 16 * i
        sorte, j = partie[e], partie[e + 1]
        dec, lon = struct.unpack_from("<II", partie, e + 4)
        out[(sorte, j)] = (dec, lon)
    return out


class SourceSynth:
    """A layer generated in memory by the encoder (parts, tables) with its seeded bf16 router."""

    def __init__(self, graine, indice, E, dims, N_delta, N_codes, n_fils):
        import numpy as np

        from troncons_amd import codeur
        self.h = codeur.CoucheSynthetique(graine, indice, E, dims, N_delta=N_delta, N_codes=N_codes, n_fils=n_fils)
        r = np.stack([codeur.synth_normale_bf16(graine + indice, 3, e, dims.colonnes[0], 0.02) for e in range(E)])
        self.r16 = (r.view(np.uint32) >> 16).astype(np.uint16)
        self.taille, self.utiles, self.partie, self.freqs = self.h.taille, self.h.utiles, self.h.partie, self.h.freqs

    def liberer(self):
        self.h.liberer()


class SourceFichier:
    """One layer of an opened .trc file, read the way the reference scheduler reads it
    (trc-ordo/src/lib.rs:265-273, 389-420, 746-760): LUT frequencies from TABLES, each part read
    with its directory fingerprint and structure checked, the router from RÉSIDENTS."""

    def __init__(self, fichier, couche, E):
        import numpy as np
        self.f, self.c = fichier, couche
        self.entrees = [fichier.entree(couche, e) for e in range(E)]
        (r,) = [r for r in fichier.residents() if r.nom == f"blk.{couche}.ffn_gate_inp.weight"]
        assert r.type_ggml == 30 and r.ne[1] == E, "router resident: bf16, one row per expert"
        self.r16 = fichier.donnees_resident(r).view(np.uint16).reshape(E, -1)

    def taille(self, e):
        return self.entrees[e].longueur[0]

    def utiles(self, e):
        return self.entrees[e].utiles[0]

    def partie(self, e, dst=None):
        return self.f.lire_partie(self.c, e, dst=dst)

    def freqs(self):
        return self.f.freqs_couche(self.c)

    def liberer(self):
        pass


def ouvrir_fichier(args, E, k, dims, n_couches, n_fils):
    """Opens --fichier, writing it first (the synthetic model, one layer at a time) if it is absent."""
    from troncons_amd import conteneur
    chemin = pathlib.Path(args.fichier)
    t_ecr = 0.0
    if not chemin.exists():
        t = time.perf_counter()
        conteneur.synth_fichier(chemin, args.graine, n_couches, E, k, dims, N_delta=args.n_delta,
                                N_codes=args.n_codes, n_fils=n_fils)
        t_ecr = time.perf_counter() - t
        print(f"bench: wrote {chemin} ({chemin.stat().st_size / 1e9:.2f} GB, {t_ecr:.1f} s)", file=sys.stderr,
              flush=True)
    t = time.perf_counter()
    f = conteneur.Fichier.ouvrir(chemin)
    t_ouv = time.perf_counter() - t
    e = f.entete()
    attendu = (n_couches, E, k, args.graine, args.n_delta, args.n_codes)
    lu = (e.couches, e.experts, e.k, f.paire("troncons.synth.graine").entier(),
          f.paire("troncons.synth.pas_delta").entier(), f.paire("troncons.synth.pas_codes").entier())
    assert lu == attendu, f"{chemin}: (layers, experts, k, seed, N_delta, N_codes) = {lu}, expected {attendu}"
    assert list(e.lignes[:3]) == list(dims.lignes) and list(e.colonnes[:3]) == list(dims.colonnes)
    info = {"path": str(chemin), "bytes": int(e.taille_fichier), "write_s": round(t_ecr, 1),
            "open_s": round(t_ouv, 4), "opened_bytes_read": f.octets_lus_a_l_ouverture()}
    return f, info


class CoucheResidente:
    """One layer resident on the device: the experts' parts in one allocation (each 256-byte
    aligned), their address table, the mounted directory, the layer LUTs and the router."""

    def __init__(self, source, E, dims, dev, fz, flux):
        import numpy as np
        import torch

        from troncons_amd import fusion
        from troncons_amd import noyaux as K
        from troncons_amd.noyaux import VueCarte

        t = time.perf_counter()
        self.hote = source
        tailles = [self.hote.taille(e) for e in range(E)]
        self.utiles = np.array([self.hote.utiles(e) for e in range(E)], np.int64)
        self.decal = np.concatenate([[0], np.cumsum(tailles)[:-1]]).astype(np.int64)
        self.bloc = torch.empty(int(sum(tailles)) + 256, dtype=torch.uint8, device=dev)
        self.o0 = (-self.bloc.data_ptr()) % 256
        base = self.bloc.data_ptr() + self.o0
        self.octets_codes = np.zeros((E, 3), np.int64)   # CODES_CTX stream bytes per matrix
        self.octets_echelles = np.zeros((E, 3), np.int64)  # DELTA + MEDIANES stream bytes per matrix
        self.octets_matrice = np.zeros((E, 3), np.int64)  # the 4 streams of the matrix + headers
        for e in range(E):
            p = self.hote.partie(e)
            off = int(self.decal[e]) + self.o0
            self.bloc[off:off + p.size].copy_(torch.from_numpy(p))
            fl = lire_flux(p[:64 + 16 * 12].tobytes())
            for j in range(3):
                self.octets_codes[e, j] = fl[(4, j)][1]
                self.octets_echelles[e, j] = fl[(3, j)][1] + fl[(1, j)][1]
                self.octets_matrice[e, j] = 64 + 4 * 16 + sum(fl[(s, j)][1] for s in (1, 2, 3, 4))
        self.table = torch.from_numpy(np.array([base + int(d) for d in self.decal], np.uint64).view(np.int64)).to(dev)
        freqs = self.hote.freqs()
        self.luts_np = K.luts_couche([[freqs[j][t] for t in range(4)] for j in range(3)])
        self.luts = torch.from_numpy(self.luts_np.view(np.int32)).to(dev)
        self.r16 = torch.from_numpy(np.ascontiguousarray(self.hote.r16).view(np.int16)).to(dev)
        # mount once: every part parsed into the device directory of stream locations
        self.rep = torch.zeros(fusion.taille_repertoire(E), dtype=torch.uint8, device=dev)
        ctl = torch.zeros(4, dtype=torch.int32, device=dev)
        V = VueCarte.de
        fz.monter_couche(V(self.table), E, dims, V(self.rep), V(ctl), f=flux)
        torch.cuda.synchronize()
        assert (ctl.cpu().numpy() == 0).all(), f"mount control words {ctl.cpu().numpy()}"
        self.vrep, self.vluts, self.vr16 = V(self.rep), V(self.luts), V(self.r16)
        self.t_charge = time.perf_counter() - t

    def vue_partie(self, e):
        from troncons_amd.noyaux import VueCarte
        return VueCarte.de(self.bloc, int(self.decal[e]) + self.o0, int(self.hote.taille(e)))


def planifier(selections, n: int, distance: int) -> list:
    """n token indices of the sweep (selections: [tokens][k] experts, as routed by the layer) in
    sweep order, cycling, a token being taken only if none of its experts appears in the previous
    `distance` taken tokens; when a whole cycle of the sweep offers none, the constraint is relaxed
    for that step (the next token in order is taken)."""
    T = len(selections)
    derniere: dict = {}
    plan: list = []
    t = 0
    while len(plan) < n:
        pris = False
        for essai in range(T):
            c = (t + essai) % T
            if all(len(plan) - derniere.get(int(e), -10**9) > distance for e in selections[c]):
                pris = True
                break
        if not pris:
            c = t % T
        for e in selections[c]:
            derniere[int(e)] = len(plan)
        plan.append(c)
        t = c + 1
    return plan


def description_hote() -> dict:
    """The host the CPU baseline runs on: CPU model, logical CPUs, the CPUs this process may use."""
    modele = None
    try:
        for ligne in pathlib.Path("/proc/cpuinfo").read_text().splitlines():
            if ligne.startswith("model name"):
                modele = ligne.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    utilisables = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"cpu_model": modele, "nproc": os.cpu_count(), "usable_cpus": utilisables}


def baseline_cpu(couche, luts, selections, budget_s: float, n_fils: int):
    """The reference's CPU path on this host: decoder_matrice_v10 (rANS DELTA + CODES_CTX) then the
    scalar f32 MXFP4 GEMV in the reference's order, SwiGLU and the ordered combine, over the first
    timed tokens (selections: (experts, weights, x) per token). Timed twice on a steady clock: one
    thread until ~budget_s / 2 of work, then every (token, expert) of as many tokens on n_fils threads
    (the experts of a token and the tokens are independent; the reference decoder walks a stream's
    tiles in order, as the oracle does, so no tile-parallel variant is timed)."""
    sys.path.insert(0, str(RACINE / "tests"))
    import numpy as np
    import oracle_ffi as O
    from concurrent.futures import ThreadPoolExecutor

    # the parts are fetched before the clock starts: the baseline times decode and compute, not reads
    parts = {e: bytes(couche.partie(e)) for e in sorted({int(e) for idx, _w, _x in selections for e in idx})}
    d = [O.disposition_j([2880] * 3, [2880] * 3, j) for j in range(3)]

    def expert(e, x):
        slot, ctl = O.decoder_expert(parts[int(e)], luts, [2880] * 3, [2880] * 3)
        g = O.gemv_mxfp4(slot[d[0].base:d[0].base + d[0].pas], x, 2880, 2880)
        u = O.gemv_mxfp4(slot[d[1].base:d[1].base + d[1].pas], x, 2880, 2880)
        a = O.swiglu_oai(g, u)
        return O.gemv_mxfp4(slot[d[2].base:d[2].base + d[2].pas], a, 2880, 2880)

    def jeton(t):
        idx, w, x = selections[t]
        s = [expert(e, x) for e in idx]
        return O.combiner(np.zeros(2880, np.float32), np.concatenate(s), 2880, w, len(idx), 2880)

    t0 = time.perf_counter()
    n1 = 0
    octets1 = 0
    temps1 = []
    while n1 < len(selections) and (time.perf_counter() - t0) < budget_s / 2:
        ti = time.perf_counter()
        jeton(n1)
        temps1.append(time.perf_counter() - ti)
        octets1 += sum(couche.utiles(int(e)) for e in selections[n1][0])
        n1 += 1
    dt1 = time.perf_counter() - t0
    # all cores: (token, expert) tasks of up to len(selections) tokens on n_fils threads, then the
    # combines; as many tokens as fit in the other half of the budget at the measured rate
    n_tok = max(1, min(len(selections), int(n_fils * (budget_s / 2) / (dt1 / n1))))
    taches = [(t, q) for t in range(n_tok) for q in range(len(selections[t][0]))]
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=n_fils) as ex:
        sorties = list(ex.map(lambda tq: expert(selections[tq[0]][0][tq[1]], selections[tq[0]][2]), taches))
    for t in range(n_tok):
        k = len(selections[t][0])
        s = [sorties[i] for i, (tt, _q) in enumerate(taches) if tt == t]
        O.combiner(np.zeros(2880, np.float32), np.concatenate(s), 2880, selections[t][1], k, 2880)
    dtn = time.perf_counter() - t0
    octetsn = sum(couche.utiles(int(e)) for t in range(n_tok) for e in selections[t][0])
    return {
        "value": round(dtn / n_tok * 1e6, 1), "unit": "us/token", "cores": n_fils, "kind": "port",
        "gbps_compressed": round(octetsn / dtn / 1e9, 4),
        "sample": f"{n_tok} timed tokens x 4 experts as independent tasks on {n_fils} threads "
                  "(decode DELTA+CODES_CTX, f32 GEMV x3, SwiGLU), then the ordered combines",
        "single_core": {"value": round(dt1 / n1 * 1e6, 1), "unit": "us/token", "cores": 1,
                        "gbps_compressed": round(octets1 / dt1 / 1e9, 4),
                        "median_token_us": round(float(np.median(temps1)) * 1e6, 1),
                        "worst_token_us": round(float(np.max(temps1)) * 1e6, 1),
                        "sample": f"{n1} timed tokens x 4 experts, one thread"},
        "host": description_hote(),
    }


def baseline_cpu_prefill(couche, luts, x_tok, idx, budget_s: float):
    """The reference's CPU path for a prefill batch, timed on a sample and scaled: one
    decoder_matrice_v10 of every distinct chosen expert, then per (position, slot) the f32 GEMV chain
    (gate, up, SwiGLU, down) in the reference's order; single thread."""
    sys.path.insert(0, str(RACINE / "tests"))
    import numpy as np
    import oracle_ffi as O
    d = [O.disposition_j([2880] * 3, [2880] * 3, j) for j in range(3)]
    distincts = sorted(set(int(e) for e in idx.reshape(-1)))
    t0 = time.perf_counter()
    slots = {}
    for e in distincts:
        slots[e], _ = O.decoder_expert(bytes(couche.partie(e)), luts, [2880] * 3, [2880] * 3)
        if time.perf_counter() - t0 > budget_s / 3:
            break
    t_dec = (time.perf_counter() - t0) / len(slots)
    t0 = time.perf_counter()
    n = 0
    for i in range(idx.shape[0]):
        for q in range(idx.shape[1]):
            e = int(idx[i, q])
            if e not in slots:
                continue
            sl = slots[e]
            g = O.gemv_mxfp4(sl[d[0].base:d[0].base + d[0].pas], x_tok[i % len(x_tok)], 2880, 2880)
            u = O.gemv_mxfp4(sl[d[1].base:d[1].base + d[1].pas], x_tok[i % len(x_tok)], 2880, 2880)
            O.gemv_mxfp4(sl[d[2].base:d[2].base + d[2].pas], O.swiglu_oai(g, u), 2880, 2880)
            n += 1
            if time.perf_counter() - t0 > 2 * budget_s / 3:
                break
        if time.perf_counter() - t0 > 2 * budget_s / 3:
            break
    t_chaine = (time.perf_counter() - t0) / max(n, 1)
    total = len(distincts) * t_dec + idx.size * t_chaine
    return {
        "value": round(total * 1e6, 1), "unit": "us/batch", "cores": 1, "kind": "port",
        "tokens_per_s": round(idx.shape[0] / total, 2),
        "sample": f"{len(slots)} expert decodes ({t_dec * 1e3:.0f} ms each) and {n} GEMV chains "
                  f"({t_chaine * 1e3:.1f} ms each), scaled to {len(distincts)} decodes + {idx.size} chains",
    }


def bench_prefill(args, c0, dims, E, k, C, fz, flux, dev, espace, x_tok, n_fils, t_gen):
    """Config 5: one batched prefill of `positions` tokens through the resident layer."""
    import numpy as np
    import torch

    from troncons_amd import codeur, fusion
    from troncons_amd.noyaux import VueCarte
    V = VueCarte.de
    T = args.positions
    idx, w = codeur.routage_zipf(args.graine + 5, T, E, k)
    xs = np.stack([codeur.synth_normale_bf16(args.graine, 6, t, C, 1.0) for t in range(T)])
    xd = torch.from_numpy(xs).to(dev)
    idd = torch.from_numpy(idx.view(np.int32)).to(dev)
    wd = torch.from_numpy(w).to(dev)
    res = torch.zeros((T, C), dtype=torch.float32, device=dev)
    ctl = torch.zeros(4, dtype=torch.int32, device=dev)
    _tr, tr = espace(fusion.taille_travail_prefill(dims, E, T, k, args.n_codes))

    def pas(s):
        fz.prefill_moe(c0.vrep, E, c0.vluts, dims, V(xd), T, V(idd), V(wd), k, V(res), V(ctl), tr,
                       args.n_delta, args.n_codes, f=flux)

    ms = temps(pas, args.steps, args.warmup, flux)
    assert (ctl.cpu().numpy() == 0).all(), f"control words {ctl.cpu().numpy()}"
    us = ms * 1e3 / args.steps
    o = tr.adresse - _tr.data_ptr()  # the workspace starts with the piece counters (x, act)
    pieces = _tr[o:o + 8].cpu().numpy().view(np.uint32)
    noyaux = chrono_passes(fusion, pas, min(args.steps, 10))
    kern = {nom: round(v[0] / v[1] * 1e3, 2) for nom, v in noyaux.items()}
    comptes = np.bincount(idx.reshape(-1), minlength=E)
    choisis = np.nonzero(comptes)[0]
    octets = int(c0.utiles[choisis].sum())
    octets_codes = int(c0.octets_codes[choisis].sum())
    flops = 2.0 * 3 * C * C * idx.size
    # the MFMA launches: band kernels that decode their tiles (short tiles), or that copy their bands
    # from the slots the slot decoder wrote (the bench's tile lengths)
    t_mfma = sum(v for n, v in kern.items() if n.startswith(("prefill_mfma", "prefill_bande"))) * 1e-6
    t_dec = kern.get("prefill_emplacements_delta_interne", 0.0) * 1e-6
    # slot decoder: reads the chosen experts' CODES_CTX, DELTA and MEDIANES streams, writes their
    # slots' code blocks (16 bytes) and scale bytes
    octets_dec = int(c0.octets_codes[choisis].sum() + c0.octets_echelles[choisis].sum()
                     + len(choisis) * sum(dims.lignes[j] * (dims.colonnes[j] // 32) * 17 for j in range(3)))
    trafic_dec = trafic_mesure(FICHIER_PMC_PREFILL)
    ligne = {
        "metric": f"config5 us per {T}-position prefill batch (top-{k} of {E}, Zipf 1.1)",
        "value": round(us, 1), "unit": "us/batch", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32 rANS / bf16 MFMA (MXFP4 weights exact in bf16, activations in exact bf16 pieces), f32 accumulate",
        "data": "synthetic (seeded MXFP4 law A, E8M0 in [119,125], bf16 N(0,1) activations, Zipf(1.1) routing)",
        "config": {"workload": f"config5: batched prefill, {T} positions, top-{k} of {E} gpt-oss-120b experts "
                               "(.trc v1.2 rANS-coded), each chosen expert decoded once (into its slot for tiles of "
                               "16 or more macro-steps, else band by band into LDS), grouped GEMM on MFMA", "positions": T, "experts": E, "k": k,
                   "n_codes": args.n_codes, "n_delta": args.n_delta},
        "tokens_per_s": round(T / (us * 1e-6), 1),
        "experts_decoded": int(len(choisis)),
        "per_expert_positions": {"max": int(comptes.max()), "median": float(np.median(comptes[choisis])),
                                 "min": int(comptes[choisis].min())},
        "compressed_bytes": octets,
        "gbps_compressed": round(octets / (us * 1e-6) / 1e9, 1),
        "useful_tflops": round(flops / (us * 1e-6) / 1e12, 2),
        "bf16_pieces": {"x": int(pieces[0]), "act": int(pieces[1])},
        "kernel_us": kern,
        "roofline": {
            "bound": "hbm", "kernel": "prefill_emplacements_delta_interne (the chosen experts decoded into slots)",
            "achieved": round(octets_dec / t_dec / 1e9, 1), "peak": PIC_HBM, "unit": "GB/s",
            "frac": round(octets_dec / t_dec / 1e9 / PIC_HBM, 4), "traffic": trafic_dec,
            "traffic_source": (f"{FICHIER_PMC_PREFILL.relative_to(RACINE)}: rocprofv3 --pmc FETCH_SIZE then "
                               "WRITE_SIZE per dispatch of the decoder, scaled by a 64 MiB copy kernel; not "
                               "measured in this run"),
            "bytes_per_launch": octets_dec, "avg_launch_us": round(t_dec * 1e6, 1),
            "mfma_kernels_us": round(t_mfma * 1e6, 1),
            "mfma_useful_tflops": round(flops / t_mfma / 1e12, 2) if t_mfma else None,
            "mfma_peak_tflops": 2500.0,  # dense bf16
        } if t_dec else {
            "bound": "hbm", "kernel": "prefill_mfma (gate/up launch + down launch: decode + MFMA)",
            "achieved": round(octets_codes / t_mfma / 1e9, 1) if t_mfma else None, "peak": PIC_HBM, "unit": "GB/s",
            "frac": round(octets_codes / t_mfma / 1e9 / PIC_HBM, 4) if t_mfma else None, "traffic": None,
            "mfma_useful_tflops": round(flops / t_mfma / 1e12, 2) if t_mfma else None,
            "mfma_peak_tflops": 2500.0,  # dense bf16
        },
        "setup_s": round(t_gen, 1),
    }
    ligne["cpu_baseline"] = None if args.sans_cpu else baseline_cpu_prefill(c0.hote, c0.luts_np, xs, idx,
                                                                             args.budget_cpu)
    return ligne


def bench_flux(args, E, k, C, dims, dev, flux, fz, x_tok, n_fils):
    """Config 4, streaming variant, through the native engine (csrc/diffusion.cpp): the layers' parts
    live in pinned host memory. Per layer and token: router (gemv_f32 + routeur_topk into a mapped
    mailbox) on the compute stream, one host wait (the reference scheduler's per-layer sync,
    trc-ordo/src/lib.rs:1054-1128), the k chosen parts copied on the engine's copy stream, each
    expert's fused decode and MLP (trc_expert_fusionne) started on its copy's event, then the
    ordered combine. Also timed, for the overlap: the same copies alone (hipMemcpyAsync of the
    routed parts, one stream) and the same compute alone (the routed parts already on the device)."""
    import numpy as np
    import torch

    from troncons_amd import noyaux as K
    from troncons_amd.diffusion import Diffusion
    from troncons_amd.noyaux import VueCarte
    V = VueCarte.de
    nk = K.Noyaux()
    L = args.couches
    epingles, decal, tailles, vluts, routeurs = [], [], [], [], []
    fichier, info_fichier = (ouvrir_fichier(args, E, k, dims, L, n_fils) if args.fichier else (None, None))
    t0 = time.perf_counter()
    for l in range(L):
        if fichier is None:
            h = SourceSynth(args.graine, l, E, dims, args.n_delta_m, args.n_codes_m, n_fils)
        else:
            h = SourceFichier(fichier, l, E)
        t = np.array([h.taille(e) for e in range(E)], np.int64)
        d = np.concatenate([[0], np.cumsum((t + 255) // 256 * 256)[:-1]]).astype(np.int64)
        pin = torch.empty(int(d[-1] + t[-1]), dtype=torch.uint8, pin_memory=True)
        vue_pin = pin.numpy()
        for e in range(E):
            if fichier is None:
                vue_pin[d[e]:d[e] + t[e]] = h.partie(e)
            else:  # read (and checked) straight into pinned memory, as the reference's readers do
                h.partie(e, dst=vue_pin[d[e]:d[e] + t[e]])
        freqs = h.freqs()
        luts = torch.from_numpy(K.luts_couche([[freqs[j][q] for q in range(4)] for j in range(3)]).view(np.int32)).to(dev)
        r = (np.ascontiguousarray(h.r16).astype(np.uint32) << 16).view(np.float32)
        routeurs.append(torch.from_numpy(r).to(dev))
        h.liberer()
        epingles.append(pin)
        decal.append(d)
        tailles.append(t)
        vluts.append((luts, V(luts)))
        print(f"bench: layer {l} encoded into pinned host memory ({pin.numel() / 1e9:.2f} GB)", file=sys.stderr,
              flush=True)
    t_gen = time.perf_counter() - t0
    moteur = Diffusion([(epingles[l], decal[l], tailles[l], vluts[l][1], V(routeurs[l])) for l in range(L)], E, k, dims,
                       args.n_delta, args.n_codes)
    xs = torch.from_numpy(x_tok).to(dev)
    vx = [V(xs, 4 * C * t, 4 * C) for t in range(len(x_tok))]
    residu = torch.zeros(C, dtype=torch.float32, device=dev)
    # tokens run between the two stats reads: the GPU warm-up's, the warm-up and the timed ones
    n_tok = [0]

    def pas(s):
        n_tok[0] += 1
        moteur.jeton(vx[s % len(vx)], V(residu), f=flux)

    s0 = moteur.stats()
    ms = temps(pas, args.steps, args.warmup, flux)
    s1 = moteur.stats()
    assert (moteur.controle() == 0).all(), f"control words {moteur.controle()}"
    octets_tok = (s1["octets_copies"] - s0["octets_copies"]) / n_tok[0]
    attente_couche = (s1["us_attente_routeur"] - s0["us_attente_routeur"]) / (n_tok[0] * L)
    # the routing of the timed tokens (x fixed per token: the same choices every time)
    choix = []
    for s in range(args.steps):
        choix.append([moteur.couche(l, vx[s % len(vx)], V(residu), f=flux) for l in range(L)])
    torch.cuda.synchronize()
    # copies alone: the routed parts, one stream, in the engine's order
    tmax = int(max(t.max() for t in tailles))
    arr = [torch.empty(tmax, dtype=torch.uint8, device=dev) for _ in range(k)]
    copie = torch.cuda.Stream(device=dev)

    def pas_copies(s):
        with torch.cuda.stream(copie):
            for l in range(L):
                for q, e in enumerate(choix[s % args.steps][l]):
                    n, o = int(tailles[l][e]), int(decal[l][e])
                    arr[q][:n].copy_(epingles[l][o:o + n], non_blocking=True)
        flux.wait_stream(copie)

    ms_copie = temps(pas_copies, args.steps, min(args.warmup, args.steps), flux)
    # compute alone: the same launches over the routed parts already on the device
    from troncons_amd import fusion
    presents = {}
    for s in range(args.steps):
        for l in range(L):
            for e in choix[s][l]:
                if (l, int(e)) not in presents:
                    n, o = int(tailles[l][e]), int(decal[l][e])
                    t = torch.empty(n + 256, dtype=torch.uint8, device=dev)
                    v = t[(-t.data_ptr()) % 256:][:n]
                    v.copy_(epingles[l][o:o + n])
                    presents[(l, int(e))] = v
    logits = torch.zeros(E, dtype=torch.float32, device=dev)
    idx = torch.zeros(16, dtype=torch.int32, device=dev)
    poids = torch.zeros(16, dtype=torch.float32, device=dev)
    sorties = torch.zeros(k * C, dtype=torch.float32, device=dev)
    ctl = torch.zeros(4, dtype=torch.int32, device=dev)
    n_tr = fusion.taille_travail_expert(dims, args.n_codes)
    tr_t = torch.empty(n_tr + 256, dtype=torch.uint8, device=dev)
    tr = VueCarte(tr_t.data_ptr() + (-tr_t.data_ptr()) % 256, n_tr)

    def pas_calcul(s):
        x = vx[s % len(vx)]
        for l in range(L):
            nk.gemv_f32(V(routeurs[l]), x, None, V(logits), E, C, f=flux)
            nk.routeur_topk(V(logits), E, k, V(idx), V(poids), f=flux)
            for q, e in enumerate(choix[s % args.steps][l]):
                fz.expert_fusionne(V(presents[(l, int(e))]), vluts[l][1], dims, x, V(sorties, 4 * C * q, 4 * C), V(ctl),
                                   tr, args.n_delta, args.n_codes, f=flux)
            nk.combiner(V(residu), V(sorties), C, V(poids), k, C, f=flux)

    ms_calcul = temps(pas_calcul, args.steps, min(args.warmup, args.steps), flux)
    assert (ctl.cpu().numpy() == 0).all()
    moteur.detruire()
    us, us_c, us_k = (m * 1e3 / args.steps for m in (ms, ms_copie, ms_calcul))
    recouvrement = (us_c + us_k - us) / min(us_c, us_k)
    ligne = {
        "metric": f"config4 streaming us/token for the MoE part of {L} layers (experts in pinned host memory)",
        "value": round(us, 1), "unit": "us/token", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "u32 rANS / f32 GEMV",
        "data": "synthetic (seeded MXFP4 law A, E8M0 in [119,125], bf16 N(0,1) activations, bf16 N(0,0.02) router)",
        "config": {"workload": f"config4 streaming variant, native engine (trc_diffusion): a token through {L} MoE "
                               f"layers x {E} gpt-oss-120b experts kept in pinned host memory; per layer one mailbox "
                               "wait, the 4 chosen parts copied on a side stream, each expert decoded in its fused "
                               "MLP as soon as its copy lands", "layers": L, "experts": E, "k": k,
                   "n_codes": args.n_codes, "n_delta": args.n_delta,
                   "n_codes_per_matrix": list(args.n_codes_m), "n_delta_per_matrix": list(args.n_delta_m)},
        "h2d_bytes_per_token": int(octets_tok),
        "h2d_gbps": round(octets_tok / (us * 1e-6) / 1e9, 2),
        "copies_only_us": round(us_c, 1), "h2d_gbps_copies_only": round(octets_tok / (us_c * 1e-6) / 1e9, 2),
        "compute_only_us": round(us_k, 1),
        "overlap": round(recouvrement, 3),
        "host_wait_per_layer_us": round(attente_couche, 1),
        "per_layer_us": round(us / L, 1),
        "setup_s": round(t_gen, 1),
    }
    if info_fichier is not None:
        ligne["config"]["source"] = ".trc v1.2 file: parts read with fingerprints checked into pinned memory"
        ligne["trc_file"] = info_fichier
    return ligne


def bench_ordo(args, E, k, C, dims, dev, n_fils):
    """Config 4, native streaming scheduler with the slot cache (csrc/ordo.cpp): the layers' parts
    stay in the .trc file; per layer the router's top-k goes through a mapped mailbox, the cache
    decides, misses are read from the file (pread, reader threads) into pinned memory, copied and
    decoded into VRAM slots, then the layer's MLPs run over the decoded slots (reference GEMV
    order) and the combine. Warm-up tokens fill the cache; the timed tokens follow."""
    import numpy as np
    import torch

    from troncons_amd import cache as K
    from troncons_amd import codeur
    from troncons_amd.ordo import Ordonnanceur
    L = args.couches
    if not args.fichier:
        args.fichier = f"/tmp/trc_bench_L{L}_E{E}_g{args.graine}_n{args.n_delta}-{args.n_codes}.trc"
    fichier, info_fichier = ouvrir_fichier(args, E, k, dims, L, n_fils)
    n_empl = args.emplacements or L * E
    t0 = time.perf_counter()
    o = Ordonnanceur(fichier, emplacements=n_empl, tiedes=args.tiedes, verifier=args.verifier,
                     prechargement=args.prechargement, biais_cache=args.biais_cache)
    t_creer = time.perf_counter() - t0
    n_tok = args.warmup + args.steps
    x_tok = np.stack([codeur.synth_normale_bf16(args.graine, 4, t, C, 1.0) for t in range(n_tok)])
    xs = torch.from_numpy(x_tok).to(dev)
    residu = torch.zeros(dims.lignes[2], dtype=torch.float32, device=dev)
    vx = [VueCarte_de(xs, 4 * C * t, 4 * C) for t in range(n_tok)]
    for t in range(args.warmup):
        o.jeton(vx[t], residu)
    torch.cuda.synchronize()
    c0, s0 = o.compteurs(), o.stats()
    t0 = time.perf_counter()
    for t in range(args.warmup, n_tok):
        o.jeton(vx[t], residu)
        if (t - args.warmup) % 100 == 99:
            print(f"bench: {t - args.warmup + 1} timed tokens", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    ctl = o.controle()
    assert (ctl == 0).all(), f"control words {ctl}"
    c1, s1 = o.compteurs(), o.stats()
    n = args.steps
    acces = (c1.acces() - c0.acces())
    tr = o.trace()
    sim = K.Cache(n_empl, args.tiedes)
    sim.fixer_tailles(np.array([[fichier.entree(l, e).longueur[0] for e in range(E)] for l in range(L)], np.uint64))
    accord = sim.rejouer_dans(K.Trace.de(E, tr)).tuple() == c1.tuple()
    belady = K.rejouer(K.Trace.de(E, tr), n_empl, 0, K.BELADY, K.BELADY)
    us = dt / n * 1e6
    ligne = {
        "metric": f"config4 native streaming us/token for the MoE part of {L} layers (slot cache, parts read from "
                  "the .trc file)",
        "value": round(us, 1), "unit": "us/token", "n_gpus": 1, "steps": n, "warmup": args.warmup,
        "ms_per_step": round(dt / n * 1e3, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "u32 rANS decode into slots / f32 GEMV",
        "data": "synthetic (seeded MXFP4 law A, E8M0 in [119,125], bf16 N(0,1) activations, bf16 N(0,0.02) router)",
        "config": {"workload": f"config4 streaming, native scheduler: {L} layers x {E} experts in a .trc file, "
                               f"{n_empl} decoded-expert slots in HBM ({n_empl * 13.254144e-3:.1f} GB), "
                               f"{args.tiedes} pinned warm entries, LRU", "layers": L, "experts": E, "k": k,
                   "slots": n_empl, "warm_entries": args.tiedes, "n_codes": args.n_codes, "n_delta": args.n_delta,
                   "verify_reads": bool(args.verifier), "prefetch": bool(args.prechargement),
                   "cache_bias": args.biais_cache},
        "hit_rate_vram": round((c1.succes_vram - c0.succes_vram) / acces, 4),
        "hit_rate_ram": round((c1.succes_ram - c0.succes_ram) / acces, 4),
        "disk_misses_per_token": round((c1.defauts_disque - c0.defauts_disque) / n, 3),
        "bytes_read_per_token": int((s1.octets_lus - s0.octets_lus) / n),
        "bytes_copied_per_token": int((s1.octets_copies - s0.octets_copies) / n),
        "prefetch_per_token": {"issued": round((s1.pf_emis - s0.pf_emis) / n, 3),
                               "useful": round((s1.pf_utiles - s0.pf_utiles) / n, 3),
                               "bytes": int((s1.pf_octets - s0.pf_octets) / n)},
        "host_us_per_layer": {"router_wait": round((s1.us_attente_routeur - s0.us_attente_routeur) / (n * L), 2),
                              "reads_and_sends": round((s1.us_lectures - s0.us_lectures) / (n * L), 2),
                              "issue": round((s1.us_emission - s0.us_emission) / (n * L), 2)},
        "per_layer_us": round(us / L, 2),
        "simulator_agrees": bool(accord),
        "belady_hit_rate_whole_run": round(belady.succes_vram / belady.acces(), 4),
        "lru_hit_rate_whole_run": round(c1.succes_vram / c1.acces(), 4),
        "trc_file": info_fichier, "setup_s": round(t_creer, 2),
    }
    o.detruire()
    return ligne


def bench_noyaux(args, c0, dims, E, k, C, dev, flux, x_tok):
    """The reference kernel API over decoded slots (the native scheduler's layer once every part is
    in a VRAM slot; Modele::fin_couche, trc-modele/src/lib.rs:533-553): S experts are decoded once
    into slots (trc_decoder_lot), then a step takes k of them, in rotation so that a step's slots
    come from HBM (the S slots exceed the 256 MB Infinity Cache), through trc_gemv_lot over the 2k
    gate/up matrices, trc_swiglu_oai, trc_gemv_lot over the k down matrices and trc_combiner. The
    two batched GEMVs are timed by events around each launch over the same steps."""
    import numpy as np
    import torch

    from troncons_amd import noyaux as K
    N = K.Noyaux()
    V = K.VueCarte.de
    S = max(args.emplacements or 32, k)
    te = K.taille_emplacement(dims)
    R, D = dims.lignes[0], dims.lignes[2]
    pas_e = (te + 255) // 256 * 256
    slots = torch.empty(S * pas_e + 256, dtype=torch.uint8, device=dev)
    base = slots.data_ptr() + (-slots.data_ptr()) % 256
    ctl = torch.zeros(4 * S, dtype=torch.int32, device=dev)
    dd = b"".join(K.DescDecodage(c0.vue_partie(e).adresse, base + s * pas_e, c0.luts.data_ptr(),
                                 ctl.data_ptr() + 16 * s).octets() for s, e in enumerate(range(S)))
    descs_dec = torch.from_numpy(np.frombuffer(dd, np.uint8).copy()).to(dev)
    t = time.perf_counter()
    N.decoder_lot(V(descs_dec, 0, len(dd)), S, dims, f=flux)
    torch.cuda.synchronize()
    t_dec = time.perf_counter() - t
    assert (ctl.cpu().numpy() == 0).all(), "slot decode control words"
    disp = [K.disposition(dims, j) for j in range(3)]
    xs = torch.from_numpy(x_tok).to(dev)
    g = torch.zeros(k * R, dtype=torch.float32, device=dev)
    u = torch.zeros_like(g)
    a = torch.zeros_like(g)
    sorties = torch.zeros(k * D, dtype=torch.float32, device=dev)
    residu = torch.zeros(D, dtype=torch.float32, device=dev)
    poids = torch.full((k,), 1.0 / k, dtype=torch.float32, device=dev)
    n_rot = S // k
    T = x_tok.shape[0]

    def descs_pour(r, tok):
        gu, bas = [], []
        for i in range(k):
            sl = base + ((r * k + i) % S) * pas_e
            x = xs.data_ptr() + 4 * C * tok
            gu.append(bytes(K.DescGemv(sl + disp[0].base, x, g.data_ptr() + 4 * R * i, R, C)))
            gu.append(bytes(K.DescGemv(sl + disp[1].base, x, u.data_ptr() + 4 * R * i, R, C)))
            bas.append(bytes(K.DescGemv(sl + disp[2].base, a.data_ptr() + 4 * R * i, sorties.data_ptr() + 4 * D * i,
                                        D, R)))
        return b"".join(gu) + b"".join(bas)

    dg = b"".join(descs_pour(r, r % T) for r in range(n_rot))
    descs = torch.from_numpy(np.frombuffer(dg, np.uint8).copy()).to(dev)
    pas_d = 3 * k * 32
    ev = []

    def pas(s, chrono=False):
        r = s % n_rot
        o = r * pas_d
        e0 = torch.cuda.Event(enable_timing=True) if chrono else None
        if chrono:
            e0.record(flux)
        N.gemv_lot(V(descs, o, 2 * k * 32), 2 * k, R, f=flux)
        if chrono:
            e1 = torch.cuda.Event(enable_timing=True)
            e1.record(flux)
        N.swiglu_oai(V(g), V(u), V(a), k * R, f=flux)
        if chrono:
            e2 = torch.cuda.Event(enable_timing=True)
            e2.record(flux)
        N.gemv_lot(V(descs, o + 2 * k * 32, k * 32), k, D, f=flux)
        if chrono:
            e3 = torch.cuda.Event(enable_timing=True)
            e3.record(flux)
            ev.append((e0, e1, e2, e3))
        N.combiner(V(residu), V(sorties), D, V(poids), k, D, f=flux)

    ms = temps(pas, args.steps, args.warmup, flux)
    evincer_caches()
    for s in range(args.steps):
        pas(s, chrono=True)
    torch.cuda.synchronize()
    gu_us = float(np.mean([e0.elapsed_time(e1) for e0, e1, _e2, _e3 in ev])) * 1e3
    bas_us = float(np.mean([e2.elapsed_time(e3) for _e0, _e1, e2, e3 in ev])) * 1e3
    # the reference's own throughput case (banc_k's gemv_mxfp4_lot): the 3k matrices of k experts
    # as one batch of independent products, each against the token's x
    d12 = b"".join(bytes(K.DescGemv(base + ((r * k + i) % S) * pas_e + disp[j].base, xs.data_ptr() + 4 * C * (r % T),
                                    sorties.data_ptr() + 4 * D * i, dims.lignes[j], dims.colonnes[j]))
                   for r in range(n_rot) for i in range(k) for j in range(3))
    descs12 = torch.from_numpy(np.frombuffer(d12, np.uint8).copy()).to(dev)
    evincer_caches()
    ev12 = []
    for s in range(args.steps):
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record(flux)
        N.gemv_lot(V(descs12, (s % n_rot) * 3 * k * 32, 3 * k * 32), 3 * k, max(dims.lignes), f=flux)
        a1.record(flux)
        ev12.append((a0, a1))
    torch.cuda.synchronize()
    lot_us = float(np.mean([a0.elapsed_time(a1) for a0, a1 in ev12])) * 1e3
    octets_mat = disp[0].pas  # one matrix of the slot: codes, scales, biases
    o_gu, o_bas = 2 * k * octets_mat, k * octets_mat
    us = ms / args.steps * 1e3
    return {
        "metric": "reference kernel API over decoded slots: us per layer step (k experts), batched MXFP4 GEMV GB/s",
        "value": round(us, 2), "unit": "us/step", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 5), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32 GEMV over MXFP4 slots (reference operation order)",
        "data": "synthetic (seeded MXFP4 law A, E8M0 in [119,125], bf16 N(0,1) activations)",
        "config": {"workload": f"{S} gpt-oss experts decoded once into VRAM slots ({S * te / 1e9:.2f} GB); a step: "
                               f"trc_gemv_lot over {2 * k} gate/up matrices, trc_swiglu_oai, trc_gemv_lot over "
                               f"{k} down matrices, trc_combiner; {k} slots per step in rotation", "slots": S, "k": k},
        "gemv_lot_us": {"gate_up": round(gu_us, 2), "down": round(bas_us, 2),
                        "method": "CUDA events around each launch on the launch's stream (includes the launch gap)"},
        "gemv_lot_bytes": {"gate_up": o_gu, "down": o_bas},
        "gemv_lot_gbps": {"gate_up": round(o_gu / gu_us / 1e3, 1), "down": round(o_bas / bas_us / 1e3, 1)},
        "gemv_lot_frac_hbm": {"gate_up": round(o_gu / gu_us / 1e3 / PIC_HBM, 4),
                              "down": round(o_bas / bas_us / 1e3 / PIC_HBM, 4)},
        "gemv_lot_all_matrices": {"matrices": 3 * k, "bytes": 3 * k * octets_mat, "us": round(lot_us, 2),
                                  "gbps": round(3 * k * octets_mat / lot_us / 1e3, 1),
                                  "frac_hbm": round(3 * k * octets_mat / lot_us / 1e3 / PIC_HBM, 4),
                                  "method": "one trc_gemv_lot over the 3k matrices of k slots (independent "
                                            "products, as the reference's banc_k times gemv_mxfp4_lot), events"},
        "slot_decode_s": round(t_dec, 3),
    }


def VueCarte_de(t, decalage, octets):
    from troncons_amd.noyaux import VueCarte
    return VueCarte.de(t, decalage, octets)


def chrono_passes(fusion, pas, n):
    """Per-kernel durations over n steps: every kernel launched with the start/stop events that the
    runtime records at the kernel's own start and end (hipExtLaunchKernel). Kept out of the timed
    region, so that `value` carries no timing machinery."""
    import torch
    fusion.chrono(True)
    fusion.chrono_recolter(True)
    for s in range(n):
        pas(s)
    torch.cuda.synchronize()
    noyaux = fusion.chrono_recolter(True)
    fusion.chrono(False)
    return noyaux


VOCAB_GPT = 201088


def bench_modele(args, dims, flux):
    """Config 6: a whole decode step of a gpt-oss-120b-shaped model held resident — embedding row,
    36 layers (Q8_0 attention with sinks and YaRN, even layers windowed on a ring of 128, f16 KV
    cache; then the fused compressed MoE layer), the 201088-row Q8_0 head and argmax — issued by the
    native driver (csrc/modele.cpp, one call per token). Synthetic weights; positions 0, 1, ... of a seeded token
    sequence (teacher forced, so every step does the same work as a real one)."""
    import numpy as np

    from troncons_amd import modele as Mo
    from troncons_amd.noyaux import ParamsRope
    h = Mo.Hyper(couches=args.couches, d=C_GPT, tetes=64, tetes_kv=8, experts=args.experts, actifs=args.k,
                 vocab=VOCAB_GPT, eps=1e-5, rope=ParamsRope.gpt_oss(), fenetre=128, contexte=4096, dims=dims,
                 n_delta=args.n_delta, n_codes=args.n_codes, n_delta_gu=args.n_delta_gu, n_codes_gu=args.n_codes_gu)
    if args.steps + args.warmup > h.contexte:
        raise SystemExit(f"--steps + --warmup above the context of {h.contexte} positions")
    t0 = time.perf_counter()
    m = Mo.Modele.synthetique(h, args.graine, f=flux, progres=lambda l: print(
        f"bench: layer {l} encoded, uploaded and mounted ({time.perf_counter() - t0:.1f} s)", file=sys.stderr,
        flush=True))
    t_gen = time.perf_counter() - t0
    jetons = np.random.default_rng(args.graine).integers(0, h.vocab, args.steps + args.warmup)
    position = [0]

    def pas(_s):
        m.pas_natif(int(jetons[position[0]]), position[0])
        position[0] += 1

    # the GPU warm-up runs position 0 over and over (its KV slot is written again by the first
    # real step), so that the warm-up and timed steps keep their positions
    ms = temps(pas, args.steps, args.warmup, flux, chauffe=lambda n: m.pas_natif(int(jetons[0]), 0))
    ctl = m.controles_natif()
    assert (ctl == 0).all(), f"control words {ctl}"
    us = ms * 1e3 / args.steps
    q8 = lambda r, c: r * (c // 32) * 34
    attention = h.couches * (q8(h.dq, h.d) + 2 * q8(h.dkv, h.d) + q8(h.d, h.dq))
    tete = q8(h.vocab, h.d) + q8(1, h.d)
    parties = float(np.mean([t.numel() for t in m.c[0]["parties"]]))
    experts = h.couches * h.actifs * parties
    return {
        "metric": f"config6 us/token for a whole decode step of {h.couches} layers", "value": round(us, 2),
        "unit": "us/token", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms / args.steps, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "Q8_0 / f16 KV / u32 rANS / f32 GEMV", "tokens_per_s": round(1e6 / us, 1),
        "data": "synthetic (seeded Q8_0 attention and head, f32 norms, biases and sinks, bf16 router, "
                "rANS-coded MXFP4 experts)",
        "config": {"workload": f"config6: embedding, {h.couches} layers (Q8_0 attention, 64/8 heads, sinks, YaRN, "
                               "even layers windowed on 128, f16 KV; fused compressed MoE top-4 of 128), "
                               f"{h.vocab}-row Q8_0 head, argmax", "layers": h.couches, "hidden": h.d,
                   "experts": h.experts, "k": h.actifs, "vocab": h.vocab, "n_codes": h.n_codes,
                   "n_delta": h.n_delta, "n_codes_per_matrix": list(args.n_codes_m),
                   "n_delta_per_matrix": list(args.n_delta_m), "positions": f"0..{args.steps + args.warmup - 1}"},
        "bytes_per_token": {"attention_q8_0": int(attention), "head_q8_0": int(tete),
                            "experts_compressed_estimate": int(experts)},
        "gbps_effective": round((attention + tete + experts) / (us * 1e-6) / 1e9, 1),
        "roofline": None, "cpu_baseline": None, "setup_s": round(t_gen, 1),
    }


def evincer_caches():
    """A 2 x 512 MiB device copy: evicts the Infinity Cache (256 MB) and the L2s before a timed region."""
    import torch
    t = torch.empty(2 * (512 << 20), dtype=torch.uint8, device="cuda:0")
    t[512 << 20:].copy_(t[:512 << 20])
    torch.cuda.synchronize()
    del t


# Untimed GPU time spent on steps before the warm-up steps of a measurement. A short run (the
# driver's 20 steps after 5) otherwise starts at the clocks of a GPU that was idle during the
# set-up: measured on one box, 20 timed steps after 5 warm-up steps took 68.2-68.4 us/token with
# every kernel 6-7 % slower, against 64.7 after 200 warm-up steps and 65.0 for 200 timed steps.
CHAUFFE_MS = 200.0
_chauffe = {}


def chauffer(pas, flux, ms=CHAUFFE_MS, lot=16):
    """Runs pas(0), pas(1), ... (untimed, in lots of `lot` between two events) until the GPU has spent
    `ms` milliseconds on them; records what it ran for the JSON line."""
    import torch
    n, total = 0, 0.0
    while total < ms:
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(flux)
        for _ in range(lot):
            pas(n)
            n += 1
        b.record(flux)
        torch.cuda.synchronize()
        total += a.elapsed_time(b)
    _chauffe.update(steps=n, ms=round(total, 1))


def imprimer(ligne: dict) -> None:
    """The bench's one JSON line, with the untimed GPU warm-up that preceded its measurement."""
    if _chauffe:
        ligne["clock_warmup"] = {"steps": _chauffe["steps"], "ms": _chauffe["ms"],
                                 "method": f"untimed steps until {CHAUFFE_MS:.0f} ms of GPU time, before the "
                                           "warm-up steps"}
    print(json.dumps(ligne), flush=True)


def temps(pas, steps, warmup, flux, chauffe=None):
    """Milliseconds of steps pas(0) .. pas(steps - 1) between two events on `flux`, after the GPU
    warm-up (chauffer over `chauffe`, default pas(steps + ...)), then `warmup` untimed steps
    pas(steps) .. pas(steps + warmup - 1) (other inputs than the timed ones) and a cache eviction."""
    import torch
    chauffer(chauffe if chauffe is not None else (lambda n: pas(steps + n % max(warmup, 1))), flux)
    for s in range(warmup):
        pas(steps + s)
    torch.cuda.synchronize()
    evincer_caches()
    debut, fin = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    debut.record(flux)
    for s in range(steps):
        pas(s)
    fin.record(flux)
    torch.cuda.synchronize()
    return debut.elapsed_time(fin)


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", type=int, default=3, choices=(1, 2, 3, 4, 5, 6))
    ap.add_argument("--positions", type=int, default=512, help="positions of a --config 5 prefill batch")
    ap.add_argument("--couches", type=int, default=36, help="layers of --config 4 and 6")
    ap.add_argument("--flux", action="store_true",
                    help="--config 4 variant: the experts stay in pinned host memory and the chosen ones are "
                         "copied per layer on a side stream, overlapped with the decode")
    ap.add_argument("--fichier", default=None,
                    help="load the layers from this .trc file (written first from the seeded model if absent), "
                         "as the reference engine loads them, instead of encoding them in memory")
    ap.add_argument("--ordo", action="store_true",
                    help="--config 4 variant: the native streaming scheduler with the slot cache, parts read from "
                         "the .trc file (--fichier, written first if absent)")
    ap.add_argument("--emplacements", type=int, default=0, help="--ordo: decoded-expert slots in HBM (0: all)")
    ap.add_argument("--tiedes", type=int, default=0, help="--ordo: pinned warm-RAM entries of coded parts")
    ap.add_argument("--verifier", action="store_true", help="--ordo: check every part read against its fingerprint")
    ap.add_argument("--biais-cache", type=float, default=None, dest="biais_cache",
                    help="--ordo: beta added to the router score of each expert already in VRAM for the choice of "
                         "the k (the mixing weights stay unbiased)")
    ap.add_argument("--prechargement", action="store_true",
                    help="--ordo: each layer predicts the next layer's experts (its router over the normed residual) "
                         "and reads their parts ahead")
    ap.add_argument("--noyaux", action="store_true",
                    help="the reference kernel API over decoded slots: trc_gemv_lot over a layer step's k experts "
                         "(--emplacements slots decoded once, default 32)")
    ap.add_argument("--experts", type=int, default=128)
    ap.add_argument("--k", type=int, default=4)
    ap.add_argument("--n-codes", type=int, default=16, help="macro-steps per CODES_CTX tile written by the encoder")
    ap.add_argument("--n-delta", type=int, default=1, help="macro-steps per DELTA tile written by the encoder")
    ap.add_argument("--n-codes-gu", type=int, default=None, dest="n_codes_gu",
                    help="the same for the gate and up matrices (the format stores N per stream); default for "
                         "configs 3, 4 and 6 with the default 16 / 1: 32, else --n-codes")
    ap.add_argument("--n-delta-gu", type=int, default=None, dest="n_delta_gu",
                    help="the same for the gate and up matrices; default for configs 3, 4 and 6 with the "
                         "default 16 / 1: 2, else --n-delta")
    ap.add_argument("--graine", type=int, default=2026)
    ap.add_argument("--tokens", type=int, default=1000, help="seeded activations of the sweep")
    ap.add_argument("--distance-octets", type=float, default=512e6, dest="distance_octets",
                    help="config 3: compressed bytes of other parts read between two uses of an expert")
    ap.add_argument("--sans-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--graphe", type=int, default=0, metavar="N",
                    help="configs 3 and 4: issue the timed steps as HIP graph replays of N steps each, captured "
                         "before the timed region (0: one host call per step)")
    ap.add_argument("--budget-cpu", type=float, default=12.0, help="seconds of single-thread CPU baseline work")
    ap.add_argument("--calibrer-copie", action="store_true",
                    help="also run three plain 64 MiB device copies (counter calibration under rocprofv3 --pmc)")
    args = ap.parse_args()
    # per-matrix tile lengths of the synthetic layers (gate, up, down); the API calls take the down
    # matrix's, which size the workspace and choose the launch plan
    # gate/up at 32 / 2 by default for the decode step (fewer tile starts in the larger launch; the
    # down launch keeps 16 / 1, whose tiles fill the chip's wavefronts)
    defaut_gu = args.config in (3, 4, 6) and args.n_codes == 16 and args.n_delta == 1 and not args.fichier
    if args.n_codes_gu is None:
        args.n_codes_gu = 32 if defaut_gu else args.n_codes
    if args.n_delta_gu is None:
        args.n_delta_gu = 2 if defaut_gu else args.n_delta
    args.n_codes_m = (args.n_codes_gu,) * 2 + (args.n_codes,)
    args.n_delta_m = (args.n_delta_gu,) * 2 + (args.n_delta,)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); the expert-parallel "
              "sharding across GPUs is a design, not run here.", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    from troncons_amd import codeur, fusion
    from troncons_amd.noyaux import DimsExpert, VueCarte

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    dims = DimsExpert.gpt_oss()
    E, k, C = args.experts, args.k, C_GPT
    # every CPU this process may run on (its affinity mask), up to the 16 host CPUs that the GPU
    # boxes grant each GPU: the encoder's threads and the CPU baseline's all-core leg use them all
    utilisables = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    n_fils = max(1, min(utilisables, PART_CPU_PAR_GPU))
    fz = fusion.Fusion()
    flux = torch.cuda.current_stream()
    V = VueCarte.de

    if args.config == 6:
        imprimer(bench_modele(args, dims, flux))
        return

    if args.config == 4 and args.ordo:
        imprimer(bench_ordo(args, E, k, C, dims, dev, n_fils))
        return

    if args.config == 4 and args.flux:
        x_tok = np.stack([codeur.synth_normale_bf16(args.graine, 4, t, C, 1.0) for t in range(args.tokens)])
        imprimer(bench_flux(args, E, k, C, dims, dev, flux, fz, x_tok, n_fils))
        return

    n_couches = args.couches if args.config == 4 else 1
    fichier, info_fichier = (ouvrir_fichier(args, E, k, dims, n_couches, n_fils) if args.fichier else (None, None))
    couches = []
    t_gen = 0.0
    for l in range(n_couches):
        t = time.perf_counter()
        if fichier is None:
            source = SourceSynth(args.graine, l, E, dims, args.n_delta_m, args.n_codes_m, n_fils)
        else:
            source = SourceFichier(fichier, l, E)
        t_gen += time.perf_counter() - t
        couches.append(CoucheResidente(source, E, dims, dev, fz, flux))
        t_gen += couches[-1].t_charge
        print(f"bench: layer {l} {'encoded' if fichier is None else 'read from the file'} and mounted "
              f"({t_gen:.1f} s so far)", file=sys.stderr, flush=True)
    c0 = couches[0]
    x_tok = np.stack([codeur.synth_normale_bf16(args.graine, 4, t, C, 1.0) for t in range(args.tokens)])
    if args.noyaux:
        imprimer(bench_noyaux(args, c0, dims, E, k, C, dev, flux, x_tok))
        return
    xs = torch.from_numpy(x_tok).to(dev)
    vx = [V(xs, 4 * C * t, 4 * C) for t in range(args.tokens)]
    ctl = torch.zeros(4, dtype=torch.int32, device=dev)
    vctl = V(ctl)
    if args.calibrer_copie:
        # a copy kernel of known size: FETCH_SIZE / WRITE_SIZE per dispatch should read 65536 KiB
        src = torch.ones(16 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    def espace(n):
        t = torch.empty(n + 256, dtype=torch.uint8, device=dev)
        return t, VueCarte(t.data_ptr() + ((-t.data_ptr()) % 256), n)

    if args.config in (1, 2):
        # one down_proj (config 1) or one expert MLP (config 2) per step, rotating over the experts
        if args.config == 1:
            n_tr = fusion.taille_travail_gemv(C, C, args.n_codes)
        else:
            n_tr = fusion.taille_travail_expert(dims, args.n_codes)
        _tr, tr = espace(n_tr)
        y = torch.zeros(C, dtype=torch.float32, device=dev)
        vy = V(y)

        def pas(s):
            e = s % E
            if args.config == 1:
                fz.gemv_fusionnee(c0.vue_partie(e), 2, c0.vluts, C, C, vx[s % args.tokens], vy, vctl, tr,
                                  args.n_delta, args.n_codes, f=flux)
            else:
                fz.expert_fusionne(c0.vue_partie(e), c0.vluts, dims, vx[s % args.tokens], vy, vctl, tr,
                                   args.n_delta, args.n_codes, f=flux)

        ms = temps(pas, args.steps, args.warmup, flux)
        assert (ctl.cpu().numpy() == 0).all(), f"control words {ctl.cpu().numpy()}"
        sel = np.arange(args.steps) % E
        octets = (c0.octets_matrice[sel, 2] if args.config == 1 else c0.utiles[sel]).astype(np.float64)
        noyaux = chrono_passes(fusion, pas, min(args.steps, 200))
        us = ms * 1e3 / args.steps
        nom = "one down_proj 2880x2880" if args.config == 1 else "one expert MLP (gate, up, down 2880x2880)"
        ligne = {
            "metric": f"config{args.config} us per {'matrix' if args.config == 1 else 'expert'}; "
                      "compressed-weight GB/s",
            "value": round(us, 3), "unit": "us/" + ("matrix" if args.config == 1 else "expert"), "n_gpus": 1,
            "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 5),
            "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "u32 rANS / f32 GEMV",
            "data": "synthetic (seeded MXFP4 law A, E8M0 in [119,125], bf16 N(0,1) activations)",
            "config": {"workload": f"config{args.config}: {nom}, .trc v1.2 rANS-coded, rotating over {E} experts",
                       "n_codes": args.n_codes, "n_delta": args.n_delta},
            "gbps_compressed": round(float(octets.sum() / (ms * 1e-3) / 1e9), 1),
            "compressed_bytes_per_step": int(octets.mean()),
            "kernel_us": {nom_k: round(v[0] / v[1] * 1e3, 2) for nom_k, v in noyaux.items()},
            "setup_s": round(t_gen, 1),
        }
        imprimer(ligne)
        return

    if args.config == 5:
        ligne = bench_prefill(args, c0, dims, E, k, C, fz, flux, dev, espace, x_tok, n_fils, t_gen)
        imprimer(ligne)
        return

    # configs 3 and 4: the MoE layer step (one layer, or a token through L layers)
    residu = torch.zeros(C, dtype=torch.float32, device=dev)
    vres = V(residu)
    n_sel = max(args.steps, args.tokens, 1)
    sel_i = torch.zeros((n_sel, n_couches, 8), dtype=torch.int32, device=dev)
    sel_w = torch.zeros((n_sel, n_couches, 8), dtype=torch.float32, device=dev)
    vi = [[V(sel_i, 32 * (s * n_couches + l), 32) for l in range(n_couches)] for s in range(n_sel)]
    vw = [[V(sel_w, 32 * (s * n_couches + l), 32) for l in range(n_couches)] for s in range(n_sel)]
    n_tr = fusion.taille_travail_couche(dims, E, k, args.n_codes)
    _tr, tr = espace(n_tr)

    def jeton(t, ligne, f=None):
        """Token t of the sweep through the layer(s); its selection lands in row `ligne`."""
        for l, c in enumerate(couches):
            fz.couche_moe(c.vrep, E, c.vluts, dims, c.vr16, None, vx[t], k, vres, vi[ligne][l], vw[ligne][l],
                          vctl, tr, args.n_delta, args.n_codes, f=flux if f is None else f)

    # The routing of the whole sweep, read from the product path itself (untimed), then the timed
    # schedule: tokens of the sweep in order, a token taken only if none of its experts (layer 0) was
    # used by the previous `distance` scheduled tokens, cycling over the sweep until `steps` tokens;
    # warm-up on sweep tokens outside the schedule; then a copy of 2 x 512 MiB evicts the Infinity
    # Cache (256 MB) and the L2s before the timed region, so that no part is served from a cache.
    for t in range(args.tokens):
        jeton(t, t)
    torch.cuda.synchronize()
    sel_balayage = sel_i[:args.tokens, 0, :k].cpu().numpy().astype(np.int64)
    octets_tok_moyen = float(c0.utiles[sel_balayage].sum(axis=1).mean())
    distance = max(1, int(np.ceil(args.distance_octets / octets_tok_moyen))) if n_couches == 1 else 0
    plan = planifier(sel_balayage, args.steps, distance)
    dans_plan = set(plan)
    hors_plan = [t for t in range(args.tokens) if t not in dans_plan] or list(range(args.tokens))
    chasse = torch.empty(2 * (512 << 20), dtype=torch.uint8, device=dev)

    def evincer():
        chasse[512 << 20:].copy_(chasse[:512 << 20])

    chauffer(lambda n: jeton(hors_plan[n % len(hors_plan)], (args.steps + n) % n_sel), flux)
    for s in range(args.warmup):
        jeton(hors_plan[s % len(hors_plan)], (args.steps + s) % n_sel)
    graphes = []
    if args.graphe > 0:
        # the timed steps captured ahead (the same launches, arguments and order as the host calls)
        s_cap = torch.cuda.Stream(device=dev)
        s_cap.wait_stream(flux)
        for g0 in range(0, args.steps, args.graphe):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=s_cap):
                for s in range(g0, min(g0 + args.graphe, args.steps)):
                    jeton(plan[s], s, f=s_cap)
            graphes.append(g)
        flux.wait_stream(s_cap)
    evincer()
    torch.cuda.synchronize()
    debut, fin = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    debut.record(flux)
    if graphes:
        with torch.cuda.stream(flux):
            for g in graphes:
                g.replay()
    else:
        for s in range(args.steps):
            jeton(plan[s], s)
    fin.record(flux)
    torch.cuda.synchronize()
    ms = debut.elapsed_time(fin)
    del graphes
    assert (ctl.cpu().numpy() == 0).all(), f"control words {ctl.cpu().numpy()}"
    sel = sel_i[:args.steps, :, :k].cpu().numpy()
    octets_tok = sum(couches[l].utiles[sel[:, l, :]].sum(axis=1) for l in range(n_couches))
    us_tok = ms * 1e3 / args.steps
    gbps = octets_tok.sum() / (ms * 1e-3) / 1e9
    histo = np.bincount(sel[:, 0, :].reshape(-1), minlength=E)
    distincts = np.unique(sel[:, 0, :])
    octets_distincts = int(sum(couches[l].utiles[np.unique(sel[:, l, :])].sum() for l in range(n_couches)))
    # per-token distribution: the same timed steps again after another eviction, one event per token
    evincer()
    torch.cuda.synchronize()
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    evs[0].record(flux)
    for s in range(args.steps):
        jeton(plan[s], s)
        evs[s + 1].record(flux)
    torch.cuda.synchronize()
    par_jeton = np.array([evs[s].elapsed_time(evs[s + 1]) * 1e3 for s in range(args.steps)])

    n_chrono = min(args.steps, 200 if n_couches == 1 else 20)
    evincer()
    noyaux = chrono_passes(fusion, lambda s: jeton(plan[s], s), n_chrono)
    sel_c = sel_i[:n_chrono, :, :k].cpu().numpy()
    # the CODES launches: fusion_codes (each tile's DELTA decoded in the kernel) or, for other tile
    # lengths, fusion_gemv after the DELTA pass
    gu_ms, gu_n = noyaux.get("fusion_codes/gate_up", noyaux.get("fusion_gemv/gate_up", (0.0, 1)))
    bas_ms, bas_n = noyaux.get("fusion_codes/down", noyaux.get("fusion_gemv/down", (0.0, 1)))
    nom_codes = "fusion_codes" if "fusion_codes/gate_up" in noyaux else "fusion_gemv"
    # algorithmic bytes of a launch: the CODES_CTX streams it decodes, plus, when it decodes each
    # tile's DELTA itself (fusion_codes), the DELTA and MEDIANES streams
    lus = [couches[l].octets_codes + (couches[l].octets_echelles if nom_codes == "fusion_codes" else 0)
           for l in range(n_couches)]
    octets_gu = sum(lus[l][sel_c[:, l, :]][:, :, :2].sum() for l in range(n_couches)) / gu_n
    octets_bas = sum(lus[l][sel_c[:, l, :]][:, :, 2].sum() for l in range(n_couches)) / bas_n
    duree_us = (gu_ms / gu_n + bas_ms / bas_n) * 1e3
    atteint = (octets_gu + octets_bas) / (duree_us * 1e-6) / 1e9
    trafic = trafic_mesure() if n_couches == 1 else None
    roofline = {
        "bound": "hbm",
        "kernel": ("fusion_codes_gu (gate/up launch) + fusion_codes_swiglu (down launch)" if nom_codes == "fusion_codes"
                   else "fusion_gemv (gate/up launch + down launch)"),
        "achieved": round(float(atteint), 1), "peak": PIC_HBM, "unit": "GB/s",
        "frac": round(float(atteint / PIC_HBM), 4), "traffic": trafic,
        "traffic_source": (f"{FICHIER_PMC.relative_to(RACINE)}: rocprofv3 --pmc FETCH_SIZE then WRITE_SIZE per "
                           "dispatch of the same command, scaled by a 64 MiB copy kernel; not measured in this run")
        if trafic else None,
        "bytes_per_launch": {"gate_up": int(octets_gu), "down": int(octets_bas)},
        "avg_launch_us": {"gate_up": round(gu_ms / gu_n * 1e3, 2), "down": round(bas_ms / bas_n * 1e3, 2),
                          "both": round(duree_us / 2, 2)},
    }
    chrono_us = {nom: round(v[0] / v[1] * 1e3, 2) for nom, v in noyaux.items()}
    if n_couches == 1:
        metrique, unite = METRIQUE, "us/token"
        workload = (f"config3: one MoE layer decode step, batch 1, top-{k} of {E} gpt-oss-120b experts "
                    f"(3 x 2880x2880 MXFP4, .trc v1.2 rANS-coded); {args.steps} timed tokens from a "
                    f"{args.tokens}-token seeded sweep, no expert reused within {distance} tokens")
    else:
        metrique, unite = f"config4 us/token for the MoE part of {n_couches} resident layers", "us/token"
        workload = (f"config4: a token through {n_couches} resident MoE layers x 128 gpt-oss-120b experts "
                    f"(.trc v1.2 rANS-coded, {sum(int(c.utiles.sum()) for c in couches) / 1e9:.1f} GB of parts)")
    ligne = {
        "metric": metrique, "value": round(us_tok, 3), "unit": unite, "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms / args.steps, 5), "higher_is_better": False,
        "scaling": "weak", "vs_baseline": None, "dtype": "u32 rANS / f32 GEMV",
        "data": "synthetic (seeded MXFP4 law A, E8M0 in [119,125], bf16 N(0,1) activations, bf16 N(0,0.02) router)",
        "config": {"workload": workload, "experts": E, "k": k, "hidden": C, "layers": n_couches,
                   "n_codes": args.n_codes, "n_delta": args.n_delta,
                   "n_codes_per_matrix": list(args.n_codes_m), "n_delta_per_matrix": list(args.n_delta_m),
                   "tokens": args.steps, "sweep_tokens": args.tokens, "mean_part_bytes": int(c0.utiles.mean()),
                   "issue": (f"HIP graph replays of {args.graphe} steps, captured before the timed region"
                             if args.graphe > 0 else "one host call per step (trc_couche_moe_fusionnee)")},
        "gbps_compressed": round(float(gbps), 1),
        "frac_hbm_layer": round(float(gbps / PIC_HBM), 4),
        "compressed_bytes_per_token": int(octets_tok.mean()),
        "timed_distinct_part_bytes": octets_distincts,
        "cache": ("a 2 x 512 MiB device copy evicts the Infinity Cache and the L2s before the timed region; "
                  + (f"no expert recurs within {distance} scheduled tokens "
                     f"({distance * octets_tok_moyen / 1e9:.2f} GB of other parts)" if distance else
                     "each token reads every layer's parts once")),
        "token_us": {"median": round(float(np.median(par_jeton)), 2),
                     "p90": round(float(np.percentile(par_jeton, 90)), 2),
                     "worst": round(float(par_jeton.max()), 2), "best": round(float(par_jeton.min()), 2),
                     "method": "the timed steps again after another eviction, one HIP event per token"},
        "routing_histogram": {"experts_hit": int(len(distincts)), "min": int(histo.min()),
                              "max": int(histo.max()), "mean": round(float(histo.mean()), 2)},
        "kernel_us": chrono_us,
        "roofline": roofline,
        "setup_s": round(t_gen, 1),
    }
    if info_fichier is not None:
        ligne["config"]["source"] = ".trc v1.2 file: parts read with fingerprints checked, tables, router resident"
        ligne["trc_file"] = info_fichier
    if not args.sans_cpu and n_couches == 1:
        selections = [(sel[s, 0], sel_w[s, 0, :k].cpu().numpy(), x_tok[plan[s]]) for s in range(min(args.steps, 64))]
        ligne["cpu_baseline"] = baseline_cpu(c0.hote, c0.luts_np, selections, args.budget_cpu, n_fils)
    else:
        ligne["cpu_baseline"] = None
    imprimer(ligne)


if __name__ == "__main__":
    main()
