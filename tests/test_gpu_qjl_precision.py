"""The QJL term at f32 grade in every scoring and attention kernel.

The reference forms q_proj = S q in fp32 and never rounds it (kernels/attention.py:158-167,
:453).  These cases are built so that rounding q_proj to f16 anywhere would move the scores by
a large amount, while the exact estimator is easy to evaluate:

* q_proj is set directly (integers of magnitude < 2^15, so every f32 partial sum of
  sign x q_proj is exact and an (f16 hi, f16 lo) split is exact);
* every key of a (batch, kv head) has the same codes and norms and a residual norm of 8, and
  the keys' QJL sign rows differ from the first key's by flipping whole triples of dims whose
  signed q_proj values sum to exactly zero: (a, b, -(a + b)).  So every key has the same exact
  score, while the f16 roundings of a, b and -(a + b) do not cancel.

The float64 oracle on the same planes is the bar: materialised scores to 1e-6 relative to the
score scale, and attention outputs within the usual rel-err 1e-3 / cosine 0.9999.  Each case
also checks that it is sensitive: the oracle with q_proj rounded to f16 misses the bar by at
least 10x.  Kernels covered, by shape: the head_dim-128 prefill kernel (unmasked, whose lo
fragments live in LDS, and masked), the head_dim-64 prefill kernel, the tiled kernel (head dim
96, scores mode), the bit-plane decode kernels (bits 2-3, one and two groups of 4 columns), and
the table decode kernels (bits 4, and 12 columns).  With q_proj scaled by 8 and by 2^-30 the prefill,
tiled and bit-plane kernels are held to the oracle where an unscaled f16 split would overflow or
lose its lo part.
"""

import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2, _tables
from turboquant_pytorch.kernels.attention import scores_from_prepared
from turboquant_pytorch.fused import attention_from_prepared

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL = 1e-3


def _case(**kw):
    print("case:", kw, flush=True)


def _planes(d, bits, B, hkv, sk, seed):
    """q_proj per (batch, kv head) and synthetic packed key planes, as described above."""
    rng = np.random.default_rng(seed)
    mag = 2 ** 13  # |q_proj| < 2^14 + 2^13: |sum| < 2^21, exact in f32
    ntrip = min(21, d // 6)
    x = np.zeros((B, hkv, d))
    sign_bits = np.zeros((B, hkv, sk, d), np.int64)
    for b in range(B):
        for h in range(hkv):
            s0 = rng.integers(0, 2, d)
            sg = 2 * s0 - 1
            x[b, h] = rng.integers(mag // 2, mag, d) * rng.choice([-1, 1], d)
            trips = rng.permutation(d)[:3 * ntrip].reshape(ntrip, 3)
            for t in trips:
                a1, a2 = rng.integers(mag // 2, mag, 2)
                x[b, h, t] = sg[t] * np.array([a1, a2, -(a1 + a2)])
            for k in range(sk):
                s = s0.copy()
                if k:
                    s[trips[rng.random(ntrip) < 0.5].reshape(-1)] ^= 1
                sign_bits[b, h, k] = s
    codes = np.repeat(rng.integers(0, 2 ** (bits - 1), (B, hkv, 1, d)), sk, axis=2)
    return x, codes, sign_bits


def _setup(d, bits, B, hq, hkv, sq, sk, seed=0, qscale=1.0):
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    x, codes, sign_bits = _planes(d, bits, B, hkv, sk, seed)
    x = x * qscale  # a power of two: still exact in f32
    g = hq // hkv
    rng = np.random.default_rng(seed + 1)
    q_rot16 = rng.standard_normal((B, hkv, d)).astype(np.float16)
    # every query row of a kv-head group carries the group's q_rot / q_proj
    q_rot = torch.from_numpy(np.repeat(np.repeat(q_rot16[:, :, None, None], g, 2), sq, 3).reshape(B, hq, sq, d))
    q_proj = torch.from_numpy(np.repeat(np.repeat(x.astype(np.float32)[:, :, None, None], g, 2), sq, 3).reshape(B, hq, sq, d))
    rn = np.full((B, hkv, sk), 8.0, np.float16)
    vn = np.ones((B, hkv, sk), np.float16)
    ck = {
        "packed_key_indices": torch.from_numpy(O.pack_bits(codes.reshape(-1, d), bits - 1)).view(B, hkv, sk, -1).to(DEV),
        "packed_qjl_signs": torch.from_numpy(O.pack_bits(sign_bits.reshape(-1, d), 1)).view(B, hkv, sk, -1).to(DEV),
        "residual_norm": torch.from_numpy(rn).to(DEV),
        "vec_norms": torch.from_numpy(vn).to(DEV),
        "shape": (B, hkv, sk, d),
    }
    vcodes = rng.integers(0, 2 ** bits, (B * hkv * sk, d))
    vvn = np.ones(B * hkv * sk, np.float16)
    cv = {
        "packed_indices": torch.from_numpy(O.pack_bits(vcodes, bits)).view(B, hkv, sk, -1).to(DEV),
        "vec_norms": torch.from_numpy(vvn.reshape(B, hkv, sk)).to(DEV),
        "shape": (B, hkv, sk, d),
    }
    cent16 = kc.centroids.cpu().numpy().astype(np.float16)
    coeff = O.COEFF(d)

    def oracle_scores(xq):  # [B, hq, sq, sk]
        out = np.zeros((B, hq, sq, sk))
        for b in range(B):
            for h in range(hq):
                kh = h // g
                s = O.scores_packed(q_rot16[b, kh][None], xq[b, kh][None], codes[b, kh], sign_bits[b, kh],
                                    rn[b, kh], vn[b, kh], cent16, coeff)
                out[b, h] = np.repeat(s, sq, 0)
        return out

    vals = O.value_decompress(vcodes, vvn, vc.Pi.cpu().numpy(), vc.centroids.cpu().numpy()).reshape(B, hkv, sk, d)
    return kc, vc, q_rot.to(DEV), q_proj.to(DEV), ck, cv, x, oracle_scores, vals


@pytest.mark.parametrize("d,bits,hq,hkv,sq,sk", [
    (128, 3, 32, 8, 1, 64),    # bit-plane decode scores kernel
    (128, 3, 16, 2, 1, 64),    # bit-plane decode scores kernel, two column groups
    (128, 4, 32, 8, 1, 64),    # table decode scores kernel (bits 4)
    (128, 3, 32, 8, 3, 64),    # table decode scores kernel (12 columns)
    (128, 3, 8, 2, 40, 48),    # tiled kernel, scores mode
    (96, 3, 8, 2, 40, 48),     # tiled kernel at head dim 96
])
def test_scores_qjl_term_f32_grade(d, bits, hq, hkv, sq, sk):
    _case(d=d, bits=bits, hq=hq, hkv=hkv, sq=sq, sk=sk)
    B = 2
    kc, vc, q_rot, q_proj, ck, cv, x, oracle_scores, _ = _setup(d, bits, B, hq, hkv, sq, sk, seed=d + bits + sq)
    t = _tables(kc, q_rot.device, with_qjl=True)
    got = scores_from_prepared(q_rot, q_proj, ck["packed_key_indices"], ck["packed_qjl_signs"], ck["residual_norm"],
                               ck["vec_norms"], t.cent16, bits, O.COEFF(d), hkv, sk, sk).cpu().numpy().astype(np.float64)
    ref = oracle_scores(x)
    ref16 = oracle_scores(x.astype(np.float16).astype(np.float64))
    scale = np.abs(ref).max()
    err = np.abs(got - ref).max() / scale
    err16 = np.abs(ref16 - ref).max() / scale
    print(f"scores: max err {err:.2e} of the score scale {scale:.3g}; f16 q_proj would give {err16:.2e}")
    assert err16 > 1e-5  # the case is sensitive to an f16 q_proj
    assert err < 1e-6


@pytest.mark.parametrize("d,bits,hq,hkv,sq,sk,masked", [
    (128, 3, 32, 8, 64, 48, False),  # head_dim-128 prefill, lo fragments in LDS
    (128, 2, 8, 8, 40, 48, False),
    (128, 4, 8, 2, 24, 48, False),
    (128, 3, 32, 8, 64, 48, True),   # masked prefill (one column block per wave)
    (64, 3, 12, 12, 40, 48, False),  # head_dim-64 prefill
    (96, 3, 8, 2, 40, 48, False),    # tiled kernel
    (128, 3, 32, 8, 1, 64, False),   # bit-plane decode attention
    (128, 3, 16, 2, 1, 64, False),   # bit-plane decode attention, two column groups
    (128, 2, 6, 1, 1, 64, True),     # bit-plane decode attention, bits 2, 6 columns, masked
    (128, 4, 32, 8, 1, 64, False),   # table decode attention
    (128, 3, 32, 8, 3, 64, False),   # table decode attention, 12 columns
])
def test_attention_qjl_term_f32_grade(d, bits, hq, hkv, sq, sk, masked):
    _case(d=d, bits=bits, hq=hq, hkv=hkv, sq=sq, sk=sk, masked=masked)
    B = 2
    kc, vc, q_rot, q_proj, ck, cv, x, oracle_scores, vals = _setup(d, bits, B, hq, hkv, sq, sk, seed=d + 3 * bits + sq)
    mask = torch.zeros(B, 1, sq, sk, device=DEV) if masked else None
    got = attention_from_prepared(q_rot, q_proj, kc, vc, ck, cv, mask, False, None, torch.float32).cpu().numpy()
    g = hq // hkv

    def oracle_out(s):
        out = np.zeros((B, sq, hq, d))
        for b in range(B):
            for h in range(hq):
                out[b, :, h] = O.attention(s[b, h], vals[b, h // g], 1 / math.sqrt(d))
        return out

    ref = oracle_out(oracle_scores(x))
    ref16 = oracle_out(oracle_scores(x.astype(np.float16).astype(np.float64)))
    err, err16 = O.rel_err(got, ref), O.rel_err(ref16, ref)
    print(f"attention: rel-err {err:.2e}; f16 q_proj would give {err16:.2e}")
    assert err16 > 10 * REL  # the case is sensitive to an f16 q_proj
    assert err < REL and O.cosine(got.reshape(-1), ref.reshape(-1)) > 0.9999


# q_proj outside f16's range: scaled by 8 its largest values reach ~2^17 (f16 ends at 65504);
# scaled by 2^-30 (values ~2^-17..2^-15) an unscaled split would leave hi subnormal and round lo
# away (~2^-9 relative).  The prefill and tiled kernels split q_proj after a power-of-two scale
# of their own and the bit-plane decode kernels take it as per-column fixed point, so all stay
# at f32 grade.  (Much larger scales make the scores themselves too large for f32 to resolve
# attention weights: at 2^12 they reach ~6.6e6 in log2 units, whose f32 ulp is 0.5.)  The table
# decode kernels (bits 4, or more than 8 columns) split q_proj unscaled and are not held to this.
KERNEL_CASES = [
    (128, 3, 32, 8, 64, 48, False),  # head_dim-128 prefill
    (128, 3, 32, 8, 64, 48, True),   # masked prefill
    (64, 3, 12, 12, 40, 48, False),  # head_dim-64 prefill
    (96, 3, 8, 2, 40, 48, False),    # tiled kernel
    (128, 3, 32, 8, 1, 64, False),   # bit-plane decode
    (128, 2, 8, 2, 1, 64, False),    # bit-plane decode, bits 2
    (128, 3, 16, 2, 1, 64, False),   # bit-plane decode, two column groups
    (128, 2, 6, 1, 1, 64, True),     # bit-plane decode, bits 2, 6 columns, masked attention
]


@pytest.mark.parametrize("qscale", [8.0, 2.0 ** -30])
@pytest.mark.parametrize("d,bits,hq,hkv,sq,sk,masked", KERNEL_CASES)
def test_qjl_term_extreme_query_magnitudes(d, bits, hq, hkv, sq, sk, masked, qscale):
    _case(d=d, bits=bits, hq=hq, hkv=hkv, sq=sq, sk=sk, masked=masked, qscale=qscale)
    B = 2
    kc, vc, q_rot, q_proj, ck, cv, x, oracle_scores, vals = _setup(d, bits, B, hq, hkv, sq, sk,
                                                                   seed=d + 5 * bits + sq, qscale=qscale)
    g = hq // hkv
    ref_s = oracle_scores(x)
    if not masked:
        t = _tables(kc, q_rot.device, with_qjl=True)
        got_s = scores_from_prepared(q_rot, q_proj, ck["packed_key_indices"], ck["packed_qjl_signs"],
                                     ck["residual_norm"], ck["vec_norms"], t.cent16, bits, O.COEFF(d), hkv, sk,
                                     sk).cpu().numpy().astype(np.float64)
        err_s = np.abs(got_s - ref_s).max() / np.abs(ref_s).max()
        print(f"scores: max err {err_s:.2e} of the score scale")
        assert np.isfinite(got_s).all() and err_s < 1e-6
    mask = torch.zeros(B, 1, sq, sk, device=DEV) if masked else None
    got = attention_from_prepared(q_rot, q_proj, kc, vc, ck, cv, mask, False, None, torch.float32).cpu().numpy()
    ref = np.zeros((B, sq, hq, d))
    for b in range(B):
        for h in range(hq):
            ref[b, :, h] = O.attention(ref_s[b, h], vals[b, h // g], 1 / math.sqrt(d))
    err = O.rel_err(got, ref)
    print(f"attention: rel-err {err:.2e}")
    assert np.isfinite(got).all() and err < REL
