"""Lloyd-Max codebooks and the seeded random matrices of a compressor.

These run once per compressor on the host, exactly as the reference sets its
compressors up; nothing here is on the per-token path.
"""

from __future__ import annotations

import functools
import json
import math
import os

import numpy as np
import torch


@functools.lru_cache(maxsize=None)
def lloyd_max_centroids(d: int, bits: int) -> tuple[float, ...]:
    """Lloyd-Max centroids (float64) for one rotated coordinate, modelled as N(0, 1/d).

    Follows compressors.py:72-96 (``_solve_codebook``; identical copy at
    :248-268): 2^bits centroids initialised at the cell midpoints of
    [-3.5 sigma, 3.5 sigma], cells bounded by centroid midpoints and the outer
    edges +-10.5 sigma, centroid <- E[x | cell] by adaptive quadrature, at most
    200 rounds with tolerance 1e-10.  As in the reference, the convergence test
    runs before the update, so the returned centroids are the iterate that
    preceded the first step smaller than the tolerance.
    """
    from scipy import integrate

    levels = 1 << bits
    sigma = 1.0 / math.sqrt(d)

    def density(x: float) -> float:
        return (1.0 / math.sqrt(2 * math.pi * sigma ** 2)) * math.exp(-x * x / (2 * sigma ** 2))

    def first_moment(x: float) -> float:
        return x * density(x)

    lo, hi = -3.5 * sigma, 3.5 * sigma
    cur = [lo + (hi - lo) * (k + 0.5) / levels for k in range(levels)]
    for _ in range(200):
        mids = [(cur[k] + cur[k + 1]) / 2.0 for k in range(levels - 1)]
        edges = [lo * 3] + mids + [hi * 3]
        nxt = []
        for k in range(levels):
            mass, _ = integrate.quad(density, edges[k], edges[k + 1])
            moment, _ = integrate.quad(first_moment, edges[k], edges[k + 1])
            nxt.append(moment / mass if mass > 1e-15 else cur[k])
        if max(abs(nxt[k] - cur[k]) for k in range(levels)) < 1e-10:
            break
        cur = nxt
    return tuple(cur)


_TABLE_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "codebooks.json")


@functools.lru_cache(maxsize=1)
def _codebook_table() -> dict:
    """Solved codebooks shipped with the package: {"d{d}_b{bits}": [f32 hex, ...]}."""
    try:
        with open(_TABLE_PATH) as f:
            return json.load(f)
    except OSError:
        return {}


def codebook(d: int, bits: int) -> torch.Tensor:
    """f32 centroid tensor [2^bits] (compressors.py:96).

    Head dims 32/64/128/256 at 1-4 bits come from the table the solver wrote
    (``python -m turboquant_pytorch.codebook`` regenerates it); anything else is
    solved here, which takes the quadrature loop about a second."""
    hexes = _codebook_table().get(f"d{d}_b{bits}")
    if hexes is not None:
        return torch.tensor([float.fromhex(h) for h in hexes], dtype=torch.float32)
    return torch.tensor(lloyd_max_centroids(d, bits), dtype=torch.float32)


def write_codebook_table(path: str = _TABLE_PATH) -> dict:
    """Solve the shipped (d, bits) grid and write it as f32 hex strings."""
    table = {}
    for d in (32, 64, 128, 256):
        for bits in (1, 2, 3, 4):
            c = torch.tensor(lloyd_max_centroids(d, bits), dtype=torch.float32)
            table[f"d{d}_b{bits}"] = [float(v).hex() for v in c.tolist()]
    with open(path, "w") as f:
        json.dump(table, f, indent=1)
    _codebook_table.cache_clear()
    return table


def midpoints(centroids: torch.Tensor) -> torch.Tensor:
    """f32 decision boundaries between adjacent centroids (compressors.py:62, :246)."""
    return (centroids[:-1] + centroids[1:]) / 2


_PINNED_ROTATIONS: dict[tuple[int, int], torch.Tensor] = {}


def pin_rotations(rotations: dict[tuple[int, int], torch.Tensor]) -> None:
    """Make random_rotation(d, seed) return the given f32 [d, d] matrices.

    The QR factor depends on the host's LAPACK in its last bits.  A deployment
    that must reproduce another host's rotations exactly (for instance the
    reference's, whose sha256 differ from this host's) pins them here; the
    compressors built afterwards use them."""
    for (d, seed), pi in rotations.items():
        pi = torch.as_tensor(pi, dtype=torch.float32).cpu().contiguous()
        if pi.shape != (d, d):
            raise ValueError(f"pinned rotation for d={d} seed={seed} has shape {tuple(pi.shape)}")
        _PINNED_ROTATIONS[(int(d), int(seed))] = pi


def load_rotations(path: str) -> dict[tuple[int, int], torch.Tensor]:
    """Read rotations saved as an .npz of f32 arrays named "d{d}_s{seed}" (no pickles)."""
    out = {}
    with np.load(path, allow_pickle=False) as z:
        for name in z.files:
            d, seed = (int(s[1:]) for s in name.split("_"))
            out[(d, seed)] = torch.from_numpy(np.array(z[name], dtype=np.float32))
    return out


def clear_pinned_rotations() -> None:
    _PINNED_ROTATIONS.clear()


def random_rotation(d: int, seed: int) -> torch.Tensor:
    """Haar-random orthogonal Pi from a seeded Gaussian (compressors.py:50-56).

    QR of a CPU-generated N(0,1) matrix with the column signs fixed so that R
    has a non-negative diagonal (a zero sign counts as +1), which makes the
    factor unique.  A rotation pinned with pin_rotations() is returned instead.
    """
    pinned = _PINNED_ROTATIONS.get((int(d), int(seed)))
    if pinned is not None:
        return pinned.clone()
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    g = torch.randn(d, d, generator=gen)
    q, r = torch.linalg.qr(g)
    sgn = torch.sign(torch.diagonal(r))
    sgn = torch.where(sgn == 0, torch.ones_like(sgn), sgn)
    return q * sgn.unsqueeze(0)


def gaussian_matrix(d: int, seed: int) -> torch.Tensor:
    """The d x d N(0,1) QJL projection S drawn from a CPU generator (compressors.py:65-67)."""
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    return torch.randn(d, d, generator=gen)


def split_f16(w: torch.Tensor) -> torch.Tensor:
    """f16 [2, d, d] (hi, lo) split of 1024*W, the layout the HIP kernels take."""
    w64 = w.detach().to("cpu", torch.float32) * 1024.0
    hi = w64.to(torch.float16)
    lo = (w64 - hi.float()).to(torch.float16)
    return torch.stack([hi, lo]).contiguous()


if __name__ == "__main__":
    write_codebook_table()
    print("wrote", _TABLE_PATH)
