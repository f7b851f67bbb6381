"""troncons_amd — the expert hot path of troncons on MI355X (gfx950).

rANS-coded MXFP4 expert weights (.trc v1.2) decoded on the GPU, fused with the MXFP4 GEMV, the
gpt-oss SwiGLU and the top-4 combine. The native library (libtroncons_hip.so, built in-tree by
``__graft_entry__.build()``) carries every kernel behind a C-ABI; this package is its host mirror.
"""
from .noyaux import (AUCUNE, DescDecodage, DescGemv, DimsExpert, Disposition, Erreur, ErreurHip, ErreurPilote,
                     ErreurUsage, Noyaux, VueCarte)

__all__ = ["AUCUNE", "DescDecodage", "DescGemv", "DimsExpert", "Disposition", "Erreur", "ErreurHip", "ErreurPilote",
           "ErreurUsage", "Noyaux", "VueCarte"]
