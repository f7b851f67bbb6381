"""Helpers shared by the GPU tests: device copies through torch (plumbing only), synthetic experts
coded by the product encoder, and their expected slots from the oracle."""
from __future__ import annotations

import numpy as np
import torch

import oracle_ffi as O
from troncons_amd import codeur
from troncons_amd.noyaux import DimsExpert, VueCarte

DEV = "cuda:0"


def dev(a: np.ndarray | bytes, alignement: int = 256) -> torch.Tensor:
    """Copies host bytes or an array to a fresh device buffer (u8), base aligned to 256."""
    b = np.frombuffer(a, np.uint8) if isinstance(a, (bytes, bytearray)) else np.ascontiguousarray(a).view(np.uint8).reshape(-1)
    t = torch.empty(b.size + alignement, dtype=torch.uint8, device=DEV)
    dec = (-t.data_ptr()) % alignement
    v = t[dec:dec + b.size]
    v.copy_(torch.from_numpy(b.copy()))
    v._garde = t
    return v


def zeros(n: int, alignement: int = 256) -> torch.Tensor:
    t = torch.zeros(n + alignement, dtype=torch.uint8, device=DEV)
    dec = (-t.data_ptr()) % alignement
    v = t[dec:dec + n]
    v._garde = t
    return v


def hote(t: torch.Tensor, dtype=np.uint8) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy().view(dtype)


def vue(t: torch.Tensor, decalage: int = 0, octets: int | None = None) -> VueCarte:
    return VueCarte.de(t, decalage, octets)


class Expert:
    """A synthetic expert coded into a v1.2 part, with the layer LUTs and the expected slot."""

    def __init__(self, graine: int, dims: DimsExpert, N_delta: int = 256, N_codes: int = 256, n_experts_tables=1,
                 expert: int = 0):
        self.dims = dims
        ex = [codeur.synth_expert(graine, 0, e, dims) for e in range(n_experts_tables)]
        self.blocs, self.biais = ex[expert]
        self.freqs = [codeur.tables([e[0][j] for e in ex], dims.lignes[j], dims.colonnes[j] // 32) for j in range(3)]
        self.partie, self.utiles = codeur.partie(self.blocs, self.biais, self.freqs, dims, expert=expert,
                                                 N_delta=N_delta, N_codes=N_codes)
        self.luts = O.luts_couche([[self.freqs[j][t] for t in range(4)] for j in range(3)])
        self.attendu = np.concatenate([
            O.blocs_vers_soa(self.blocs[j], dims.lignes[j], dims.colonnes[j], self.biais[j], canonique=True)
            for j in range(3)])

    def partie_brute(self):
        """The raw-file part (flag bit 2: the original bytes, no -0 fold) and its expected slot."""
        flux = []
        for j in range(3):
            R, C_ = self.dims.lignes[j], self.dims.colonnes[j]
            nb = R * (C_ // 32)
            b = self.blocs[j].reshape(nb, 17)
            qs = b[:, 1:].reshape(-1)
            flux.append((0x07, j, 0xFF, nb, b[:, 0].tobytes()))
            flux.append((0x06, j, 0xFF, 16 * nb, qs.tobytes()))
            flux.append((0x02, j, 0xFF, 4 * R, self.biais[j].astype(np.float32).tobytes()))
        p, _ = O.assembler_partie(0, 0, 0, 3, flux)
        attendu = np.concatenate([
            O.blocs_vers_soa(self.blocs[j], self.dims.lignes[j], self.dims.colonnes[j], self.biais[j], canonique=False)
            for j in range(3)])
        return p, attendu


# Doubled E2M1 magnitudes (codes 0-7; bit 3 is the sign): the reference's k table.
K_E2M1X2 = np.array([0.0, 1.0, 2.0, 3.0, 4.0, 6.0, 8.0, 12.0])


def poids_f64(blocs17: np.ndarray, R: int, C_: int) -> np.ndarray:
    """The R x C matrix of an uncompressed MXFP4 matrix (17-byte blocks: E8M0 scale, then 16 code
    bytes, byte i = weight i in its low nibble and weight 16 + i in its high one) in f64:
    k[c & 7] * (-1 if c & 8) * 2^(e - 128). Code 8 reads as 0, as in the reference."""
    b = np.asarray(blocs17, np.uint8).reshape(R * (C_ // 32), 17)
    qs = b[:, 1:]
    codes = np.empty((b.shape[0], 32), np.uint8)
    codes[:, :16] = qs & 15
    codes[:, 16:] = qs >> 4
    v = K_E2M1X2[codes & 7] * np.where(codes & 8, -1.0, 1.0)
    v *= np.ldexp(1.0, b[:, 0].astype(np.int32) - 128)[:, None]
    return v.reshape(R, C_)


def mlp_f64(blocs, biais, X: np.ndarray) -> np.ndarray:
    """gpt-oss expert MLP in f64 from uncompressed weights, for the columns of X (C x n):
    down(swiglu_oai(gate X + b_g, up X + b_u)) + b_d, SwiGLU with alpha 1.702, limit 7, up + 1."""
    R, C_ = biais[0].size, X.shape[0]
    g = poids_f64(blocs[0], R, C_) @ X + biais[0].astype(np.float64)[:, None]
    u = poids_f64(blocs[1], R, C_) @ X + biais[1].astype(np.float64)[:, None]
    g = np.minimum(g, 7.0)
    u = np.clip(u, -7.0, 7.0)
    a = g / (1.0 + np.exp(-1.702 * g)) * (u + 1.0)
    D = biais[2].size
    return poids_f64(blocs[2], D, R) @ a + biais[2].astype(np.float64)[:, None]


def carte_parallele(f, elements, fils: int = 16):
    """[f(e) for e in elements] on a thread pool (the oracle's and the generator's C calls release
    the GIL, and so does numpy's BLAS)."""
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=fils) as ex:
        return list(ex.map(f, elements))
