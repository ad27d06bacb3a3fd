"""Seeded random shapes through the scores and attention entry points, against the oracle.

The hand-picked cases elsewhere pin the boundaries each kernel was written around; this
sweep draws shapes the kernels' tiling does not line up with: GQA groups 1-8 (including
3 and 5, which leave MFMA columns unused), key counts that are not multiples of the
16/32/64-key blocks, 1-48 query rows (decode, split-K and prefill paths), causal or not,
bits 2-4, head_dim 64 and 128.  Same bar as the rest of the suite: rel-err 1e-3 and
cosine 0.9999 against the float64 oracle evaluated on the device's own packed planes.
A second set draws decode-shaped cases (1-2 query rows, head_dim 128, and a third head_dim
64) with 600-20000 keys, so the split-K decode kernels run with many splits and their merge
combines them.
"""

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from test_gpu_kernels import _oracle_attention, _oracle_scores
from turboquant_pytorch import compressed_attention
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL = 1e-3


def _shapes(n, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        d = 128 if rng.random() < 0.8 else 64
        bits = int(rng.integers(2, 5))
        hkv = int(rng.choice([1, 2, 4, 8]))
        g = int(rng.choice([1, 2, 3, 4, 5, 8]))
        sq = int(rng.choice([1, 1, 2, 3, 7, 16, 33, 48]))
        causal = bool(rng.random() < 0.6)
        sk = int(rng.integers(1, 600))
        if causal:
            sk = max(sk, sq)
        b = int(rng.integers(1, 3))
        out.append((d, bits, b, hkv * g, hkv, sq, sk, causal))
    return out


def _long_shapes(n, seed=4242):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        bits = int(rng.integers(2, 5))
        hkv = int(rng.choice([1, 2, 4, 8]))
        g = int(rng.choice([1, 2, 4, 8]))
        sq = int(rng.choice([1, 1, 2]))
        sk = int(rng.integers(600, 20000))
        causal = bool(rng.random() < 0.6)
        b = int(rng.integers(1, 3))
        out.append((128, bits, b, hkv * g, hkv, sq if g * sq <= 16 else 1, sk, causal))
    return out


def _long_shapes_d64(n, seed=6464):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        bits = int(rng.integers(2, 5))
        hkv = int(rng.choice([1, 2, 4, 12]))
        g = int(rng.choice([1, 2, 3, 4, 8, 16]))
        sq = int(rng.choice([1, 1, 2, 4]))
        sk = int(rng.integers(600, 20000))
        causal = bool(rng.random() < 0.6)
        b = int(rng.integers(1, 3))
        out.append((64, bits, b, hkv * g, hkv, sq if g * sq <= 16 else 1, sk, causal))
    return out


@pytest.mark.parametrize("d,bits,B,hq,hkv,sq,sk,causal", _shapes(24) + _long_shapes(6) + _long_shapes_d64(6))
def test_random_shape_scores_and_attention(d, bits, B, hq, hkv, sq, sk, causal):
    print("case:", dict(d=d, bits=bits, B=B, hq=hq, hkv=hkv, sq=sq, sk=sk, causal=causal), flush=True)
    torch.manual_seed(d * 7 + bits * 131 + hq * 17 + sq * 5 + sk)
    q = torch.randn(B, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)

    got_s = kc.asymmetric_attention_scores(q, ck).cpu().numpy()
    ref_s = _oracle_scores(kc, q, ck, hq, hkv)
    assert got_s.shape == ref_s.shape
    assert O.rel_err(got_s, ref_s) < REL

    got = compressed_attention(q, kc, vc, ck, cv, causal=causal, out_dtype=torch.float32).cpu().numpy()
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, causal=causal)
    assert got.shape == ref.shape
    assert O.rel_err(got, ref) < REL and O.cosine(got, ref) > 0.9999
