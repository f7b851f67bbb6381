"""Loading and building of the native library (libtroncons_hip.so, built in-tree for gfx950).

There is no fallback: if the library is missing or does not load, every entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib
import subprocess

PAQUET = pathlib.Path(__file__).resolve().parent
RACINE = PAQUET.parent
CSRC = PAQUET / "csrc"
LIB_PATH = PAQUET / "libtroncons_hip.so"

SOURCES_HIP = ["noyaux.hip", "fusion.hip", "prefill.hip", "passe.hip", "pilote.hip"]
SOURCES_CPP = ["hote.cpp", "codeur.cpp", "chrono.cpp", "conteneur.cpp", "cache.cpp", "ordo.cpp", "modele.cpp",
               "diffusion.cpp"]

# -packed-fp32-ops off: v_pk_* f32 forms are avoided on these boxes (the host pass warns that it
# does not know the feature; harmless).
DRAPEAUX = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-Xclang", "-target-feature",
            "-Xclang", "-packed-fp32-ops", "-pthread"]


def construire(verbeux: bool = False) -> pathlib.Path:
    """Compiles every source of csrc/ into libtroncons_hip.so (hipcc, gfx950)."""
    sources = [str(CSRC / s) for s in SOURCES_HIP + SOURCES_CPP if (CSRC / s).exists()]
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = ["hipcc", *DRAPEAUX, *sources, "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("hipcc a échoué :\n" + r.stderr[-8000:])
    if verbeux:
        print(" ".join(cmd))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


_lib = None


def charger() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise OSError(f"{LIB_PATH} absente : lancer __graft_entry__.build() (pas de repli sans le HIP)")
        _lib = C.CDLL(str(LIB_PATH))
    return _lib
