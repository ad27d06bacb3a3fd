"""Pin the compressor set-up (rotation, QJL matrix, Lloyd-Max codebooks).

Checks: reference golden fixtures (tests/golden/make_golden.py), Max's (1960)
Gaussian quantiser tables, the Lloyd fixed-point conditions evaluated with
closed-form Gaussian moments (independent of quadrature), and the uniqueness
of the sign-fixed QR factor.
"""

import hashlib
import json
import math
import os

import numpy as np
import pytest
import torch
from scipy.stats import norm

from turboquant_pytorch.codebook import codebook, gaussian_matrix, lloyd_max_centroids, random_rotation
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")

# Max (1960), optimum quantiser for N(0,1): positive output levels
MAX_TABLE = {
    1: [0.7979],
    2: [0.4528, 1.510],
    3: [0.2451, 0.7560, 1.344, 2.152],
    4: [0.1284, 0.3881, 0.6568, 0.9424, 1.256, 1.618, 2.069, 2.733],
}


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("d", [64, 128])
def test_codebook_matches_max_tables(d, bits):
    c = np.array(lloyd_max_centroids(d, bits)) * math.sqrt(d)
    pos = np.sort(c[c > 0])
    assert np.allclose(pos, MAX_TABLE[bits], rtol=2e-3, atol=2e-3)
    assert abs(c.sum()) < 1e-6  # symmetric (reference test_turboquant.py:32-35)


def _lloyd_closed_form(d, bits):
    """The same Lloyd iteration with conditional means from the Gaussian cdf/pdf
    (E[x | a < x < b] = sigma (phi(a) - phi(b)) / (Phi(b) - Phi(a))) instead of quadrature."""
    sigma = 1 / math.sqrt(d)
    n = 1 << bits
    cur = np.array([-3.5 * sigma + 7 * sigma * (k + 0.5) / n for k in range(n)])
    for _ in range(200):
        edges = np.concatenate([[-10.5 * sigma], (cur[:-1] + cur[1:]) / 2, [10.5 * sigma]])
        a, b = edges[:-1] / sigma, edges[1:] / sigma
        new = sigma * (norm.pdf(a) - norm.pdf(b)) / (norm.cdf(b) - norm.cdf(a))
        if np.max(np.abs(new - cur)) < 1e-10:
            break
        cur = new
    return cur


@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("d", [32, 128])
def test_codebook_matches_closed_form_lloyd(d, bits):
    c = np.array(lloyd_max_centroids(d, bits))
    assert np.max(np.abs(_lloyd_closed_form(d, bits) - c)) < 1e-9
    if bits <= 3:  # converged: a fixed point of the Lloyd map to 1e-9
        sigma = 1 / math.sqrt(d)
        edges = np.concatenate([[-10.5 * sigma], (c[:-1] + c[1:]) / 2, [10.5 * sigma]])
        a, b = edges[:-1] / sigma, edges[1:] / sigma
        cm = sigma * (norm.pdf(a) - norm.pdf(b)) / (norm.cdf(b) - norm.cdf(a))
        assert np.max(np.abs(cm - c)) < 1e-9


def test_codebook_matches_reference_bits():
    with open(os.path.join(GOLDEN, "codebooks.json")) as f:
        books = json.load(f)
    for key, rec in books.items():
        d, bits = (int(s[1:]) for s in key.split("_"))
        c = codebook(d, bits)
        assert [float(v).hex() for v in c.tolist()] == rec["centroids_hex"], key
        comp = TurboQuantCompressorMSE(d, bits, seed=0)
        assert [float(v).hex() for v in comp.boundaries.tolist()] == rec["boundaries_hex"], key


def _sha(t):
    return hashlib.sha256(t.contiguous().float().numpy().tobytes()).hexdigest()


def test_rotation_and_qjl_match_reference_hashes():
    with open(os.path.join(GOLDEN, "setup.json")) as f:
        setup = json.load(f)
    for key, rec in setup.items():
        d, seed = (int(s[1:]) for s in key.split("_"))
        kc = TurboQuantCompressorV2(d, 3, seed=seed)
        vc = TurboQuantCompressorMSE(d, 3, seed=seed + 10000)
        assert _sha(kc.Pi) == rec["key_pi"], key
        assert _sha(kc.S) == rec["key_s"], key
        assert _sha(vc.Pi) == rec["val_pi"], key
        # the key S and the value Pi of a layer come from the same Gaussian draw
        assert torch.equal(kc.S, gaussian_matrix(d, seed + 10000))


@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_rotation_is_unique_qr_factor(d):
    pi = random_rotation(d, 7).double()
    assert torch.allclose(pi @ pi.T, torch.eye(d, dtype=torch.float64), atol=1e-5)
    gen = torch.Generator().manual_seed(7)
    g = torch.randn(d, d, generator=gen).double()
    r = pi.T @ g  # = R with a non-negative diagonal
    assert torch.allclose(torch.tril(r, -1), torch.zeros_like(r), atol=1e-4)
    assert bool((torch.diagonal(r) > 0).all())


def test_package_codebook_table_is_the_solver_and_the_reference():
    """The shipped table (read at construction instead of re-solving) equals both the
    solver's output and the reference's exact f32 codebooks."""
    from turboquant_pytorch.codebook import _TABLE_PATH

    with open(_TABLE_PATH) as f:
        table = json.load(f)
    with open(os.path.join(GOLDEN, "codebooks.json")) as f:
        books = json.load(f)
    assert set(table) == set(books)
    for key, hexes in table.items():
        d, bits = (int(s[1:]) for s in key.split("_"))
        assert hexes == books[key]["centroids_hex"], key
        solved = torch.tensor(lloyd_max_centroids(d, bits), dtype=torch.float32)
        assert [float(v).hex() for v in solved.tolist()] == hexes, key


def test_pinned_rotations_replace_the_qr():
    """pin_rotations() is the fallback for a host whose LAPACK rounds the QR differently:
    the reference's rotations (tests/golden/rotations.npz) pinned, compressors reproduce
    the reference hashes whatever this host's QR gives."""
    from turboquant_pytorch.codebook import clear_pinned_rotations, load_rotations, pin_rotations

    rots = load_rotations(os.path.join(GOLDEN, "rotations.npz"))
    with open(os.path.join(GOLDEN, "setup.json")) as f:
        setup = json.load(f)
    try:
        fake = {k: torch.flip(v, dims=[0]) for k, v in rots.items()}  # a different "host QR"
        pin_rotations(fake)
        assert torch.equal(TurboQuantCompressorV2(64, 3, seed=42).Pi, fake[(64, 42)])
        pin_rotations(rots)
        for (d, seed) in rots:
            if f"d{d}_s{seed}" in setup:
                kc = TurboQuantCompressorV2(d, 3, seed=seed)
                vc = TurboQuantCompressorMSE(d, 3, seed=seed + 10000)
                rec = setup[f"d{d}_s{seed}"]
                assert _sha(kc.Pi) == rec["key_pi"] and _sha(vc.Pi) == rec["val_pi"]
        with pytest.raises(ValueError):
            pin_rotations({(64, 1): torch.zeros(3, 3)})
    finally:
        clear_pinned_rotations()
    assert _sha(random_rotation(64, 42)) == setup["d64_s42"]["key_pi"]
