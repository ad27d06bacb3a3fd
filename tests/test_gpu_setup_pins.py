"""Compressor set-up pinned on the GPU box itself.

Pi (a LAPACK QR), S (a seeded torch.randn) and the Lloyd-Max codebooks are
computed on the host of whatever machine runs the model.  These checks repeat
the set-up pins of tests/test_setup_pins.py there: the sha256 of Pi / S for
every per-layer seed the benchmark configurations use (reference
compressors.py:42-70, :230-246; seeds patch.py:62-75) and the exact f32
codebooks.  Where this host's QR rounds differently from the reference's,
the reference's rotations (tests/golden/rotations.npz) are pinned with
codebook.pin_rotations() and must then reproduce the reference hashes.
"""

import hashlib
import json
import os

import numpy as np
import pytest
import torch

from turboquant_pytorch.codebook import (clear_pinned_rotations, codebook, load_rotations, midpoints,
                                         pin_rotations)
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _sha(t):
    return hashlib.sha256(t.detach().cpu().contiguous().float().numpy().tobytes()).hexdigest()


def test_setup_hashes_on_this_host():
    print("case: set-up hashes", flush=True)
    with open(os.path.join(GOLDEN, "setup.json")) as f:
        setup = json.load(f)
    rots = load_rotations(os.path.join(GOLDEN, "rotations.npz"))
    drift = []
    for key, rec in setup.items():
        d, seed = (int(s[1:]) for s in key.split("_"))
        kc = TurboQuantCompressorV2(d, 3, seed=seed)
        vc = TurboQuantCompressorMSE(d, 3, seed=seed + 10000)
        assert _sha(kc.S) == rec["key_s"], f"{key}: S is a seeded randn and must not drift"
        for name, pi, s_ in (("key_pi", kc.Pi, seed), ("val_pi", vc.Pi, seed + 10000)):
            if _sha(pi) != rec[name]:
                drift.append((d, s_, name))
    print(f"{len(setup)} seed pairs checked; rotations that differ from the reference's: {drift}", flush=True)
    # every config seed (patch.py:62-75 from seed 42) has its reference rotation committed;
    # seed 0 is a test seed only
    missing = [(d, s) for d, s, _ in drift if (d, s) not in rots and s % 10000 >= 42]
    assert not missing, f"QR differs from the reference on this host for {missing} and no fixture pins them"
    drift = [x for x in drift if (x[0], x[1]) in rots]
    if drift:
        try:
            pin_rotations({(d, s): rots[(d, s)] for d, s, _ in drift})
            for d, s, name in drift:
                key = f"d{d}_s{s if name == 'key_pi' else s - 10000}"
                comp = TurboQuantCompressorV2(d, 3, seed=s) if name == "key_pi" else \
                    TurboQuantCompressorMSE(d, 3, seed=s)
                assert _sha(comp.Pi) == setup[key][name]
                # the hosts differ only by the f32 QR's rounding (measured up to ~2e-5 per
                # element between this container's MKL and the MI355X boxes')
                host = torch.linalg.qr(torch.randn(d, d, generator=torch.Generator().manual_seed(s)))[0]
                assert float((host.abs() - comp.Pi.abs()).abs().max()) < 1e-4
        finally:
            clear_pinned_rotations()


def test_codebooks_on_this_host():
    print("case: codebooks", flush=True)
    with open(os.path.join(GOLDEN, "codebooks.json")) as f:
        books = json.load(f)
    for key, rec in books.items():
        d, bits = (int(s[1:]) for s in key.split("_"))
        c = codebook(d, bits)
        assert [float(v).hex() for v in c.tolist()] == rec["centroids_hex"], key
        assert [float(v).hex() for v in midpoints(c).tolist()] == rec["boundaries_hex"], key
    # the device tables the kernels read are the same bits
    kc = TurboQuantCompressorV2(128, 4, seed=42, device="cuda")
    assert np.array_equal(kc.centroids.cpu().numpy(), codebook(128, 3).numpy())
