"""Pin the CPU oracle against closed forms, hand-derived known answers and brute force.

The oracle (oracle/tq_oracle.py) is the checker for the GPU kernels, so every
function it provides is checked here against something other than itself.
"""

import math

import numpy as np
import pytest

from oracle import tq_oracle as O


# ---------------------------------------------------------------- bit layout (bit_ops.py:243-326)

def test_pack_known_answers():
    # b=3, codes 1..7,0 -> bit stream LSB-first: 001 010 011 100 101 110 111 000 (per code, LSB first)
    packed = O.pack_bits(np.array([[1, 2, 3, 4, 5, 6, 7, 0]]), 3)
    # bits: c0=1 ->b0..2=1,0,0 ; c1=2 -> 0,1,0 ; c2=3 -> 1,1,0 ; c3=4 -> 0,0,1 ; c4=5 -> 1,0,1
    # c5=6 -> 0,1,1 ; c6=7 -> 1,1,1 ; c7=0 -> 0,0,0
    # byte0 = bits0..7 = 1,0,0,0,1,0,1,1 -> 0b11010001 = 0xD1
    # byte1 = bits8..15 = 0,0,0,1,1,0,1,0 -> 0b01011000 = 0x58
    # byte2 = bits16..23 = 1,0,1,1,1,1,0,0... careful: bits16..23 = c5 b1,b2 (1,1), c6 (1,1,1), c7 (0,0,0)
    assert packed.tolist() == [[0xD1, 0x58, 0x1F]]
    # b=2: four codes per byte, code i at bits 2i
    assert O.pack_bits(np.array([[3, 0, 1, 2]]), 2).tolist() == [[0b10010011]]
    # b=1: bit i of byte i//8
    assert O.pack_bits(np.array([[1, 0, 0, 0, 0, 0, 0, 1, 1]]), 1).tolist() == [[0x81, 0x01]]
    # masking to b bits (bit_ops.py:274)
    assert O.pack_bits(np.array([[5]]), 2).tolist() == [[1]]
    # b=5 straddle: code 31 at bits 0..4, code 1 at bits 5..9 -> byte0 = 0b00111111, byte1 = 0b00
    assert O.pack_bits(np.array([[31, 1]]), 5).tolist() == [[0x3F, 0x00]]


def test_pack_matches_bitwise_definition():
    rng = np.random.default_rng(3)
    for b in range(1, 9):
        for d in (1, 7, 32, 128):
            codes = rng.integers(0, 1 << b, size=(5, d))
            packed = O.pack_bits(codes, b)
            assert packed.shape == (5, math.ceil(d * b / 8))
            for r in range(5):
                stream = 0
                for i in range(d):
                    stream |= int(codes[r, i]) << (i * b)
                expect = [(stream >> (8 * k)) & 0xFF for k in range(packed.shape[1])]
                assert packed[r].tolist() == expect


@pytest.mark.parametrize("b", range(1, 9))
def test_unpack_roundtrip(b):
    rng = np.random.default_rng(42 + b)
    codes = rng.integers(0, 1 << b, size=(100, 128))
    assert np.array_equal(O.unpack_bits(O.pack_bits(codes, b), b, 128), codes)
    for val in (0, (1 << b) - 1):
        full = np.full((10, 64), val)
        assert np.array_equal(O.unpack_bits(O.pack_bits(full, b), b, 64), full)


# ---------------------------------------------------------------- quantisation rules

def test_searchsorted_rule_brute_force_and_ties():
    bounds = np.array([-0.5, 0.0, 0.25], np.float32)
    ys = np.array([-1, -0.5, -0.4999, 0.0, 1e-30, 0.25, 0.2500001, 3], np.float32)
    expect = [sum(1 for b in bounds if b < y) for y in ys]
    assert O.quantize_searchsorted(ys, bounds).tolist() == expect
    # ties land in the lower cell (side='left'): y == boundary j -> code j
    assert O.quantize_searchsorted(bounds, bounds).tolist() == [0, 1, 2]
    # one ulp above a boundary moves to the next cell
    up = np.nextafter(bounds, np.float32(np.inf))
    assert O.quantize_searchsorted(up, bounds).tolist() == [1, 2, 3]


def test_argmin_first_minimum():
    c = np.array([-1.0, 0.0, 1.0], np.float32)
    assert O.quantize_argmin(np.array([0.5, -0.5, 2.0], np.float32), c).tolist() == [1, 0, 2]


def test_dequantize_lookup():
    c = np.array([-1.5, -0.5, 0.5, 1.5], np.float32)
    packed = O.pack_bits(np.array([[0, 3, 2, 1]]), 2)
    assert O.dequantize(packed, c, 2, 4).astype(np.float32).tolist() == [[-1.5, 1.5, 0.5, -0.5]]


# ---------------------------------------------------------------- compression invariants

def _orth(d, seed):
    q, _ = np.linalg.qr(np.random.default_rng(seed).standard_normal((d, d)))
    return q.astype(np.float32)


def test_key_compress_identity_rotation_reduces_to_scalar_quantizer():
    d = 8
    pi = np.eye(d, dtype=np.float32)
    s = np.eye(d, dtype=np.float32)
    cent = np.array([-0.6, -0.2, 0.2, 0.6], np.float32)
    bounds = (cent[:-1] + cent[1:]) / 2
    x = np.array([[0.9, -0.1, 0.05, -0.3, 0.1, 0.2, -0.05, 0.3]], np.float32)
    out = O.key_compress_packed(x, pi, s, cent, bounds, 2)
    vn = np.linalg.norm(x)
    y = x / (vn + 1e-8)
    codes = [sum(1 for b in bounds if b < v) for v in y[0]]
    assert out["codes"][0].tolist() == codes
    kmse = cent.astype(np.float16).astype(np.float32)[codes] * vn
    assert np.allclose(out["k_mse"][0], kmse, atol=1e-6)
    # with S = I the projection is the residual itself
    assert np.array_equal(out["proj"][0] >= 0, (x[0] - kmse) >= 0)


def test_value_decompress_inverts_rotation():
    d = 16
    pi = _orth(d, 1)
    cent = np.linspace(-1, 1, 8).astype(np.float32)
    codes = np.random.default_rng(0).integers(0, 8, size=(3, d))
    vn = np.array([1.0, 2.0, 0.5], np.float16)
    rec = O.value_decompress(codes, vn, pi, cent)
    # rotating back with Pi^T recovers scaled centroids
    assert np.allclose(rec @ pi.astype(np.float64).T, cent[codes] * vn.astype(np.float64)[:, None], atol=1e-6)


# ---------------------------------------------------------------- estimator and attention

def test_scores_packed_matches_brute_force():
    rng = np.random.default_rng(5)
    d, nq, nk = 8, 3, 4
    cent16 = np.array([-0.3, -0.1, 0.1, 0.3], np.float16)
    qr = rng.standard_normal((nq, d)).astype(np.float16)
    qp = rng.standard_normal((nq, d))
    codes = rng.integers(0, 4, size=(nk, d))
    sb = rng.integers(0, 2, size=(nk, d))
    rn = rng.random(nk).astype(np.float16)
    vn = rng.random(nk).astype(np.float16)
    coeff = math.sqrt(math.pi / 2) / d
    got = O.scores_packed(qr, qp, codes, sb, rn, vn, cent16, coeff)
    for i in range(nq):
        for j in range(nk):
            t1 = sum(float(qr[i, t]) * float(cent16[codes[j, t]]) for t in range(d)) * float(vn[j])
            t2 = sum(qp[i, t] * (1 if sb[j, t] else -1) for t in range(d)) * coeff * float(rn[j])
            assert got[i, j] == pytest.approx(t1 + t2, rel=1e-12, abs=1e-12)


def test_estimator_is_unbiased_for_exact_keys():
    # With k_mse = 0 the estimator is sqrt(pi/2)/m * ||k|| * <Sq, sign(Sk)>, whose
    # mean over Gaussian S is <q, k> (QJL, TurboQuant paper Lemma 4).
    rng = np.random.default_rng(11)
    d, m, trials = 16, 16, 4000
    q = rng.standard_normal(d)
    k = rng.standard_normal(d)
    est = []
    for _ in range(trials):
        s = rng.standard_normal((m, d))
        est.append(O.scores_unpacked(q[None], np.zeros((1, d)), np.where(s @ k >= 0, 1, -1)[None],
                                     np.array([np.linalg.norm(k)]), s, O.COEFF(m))[0, 0])
    assert np.mean(est) == pytest.approx(q @ k, abs=4 * np.std(est) / math.sqrt(trials))


def test_attention_matches_loops():
    rng = np.random.default_rng(2)
    sq, sk, d = 3, 5, 4
    s = rng.standard_normal((sq, sk))
    v = rng.standard_normal((sk, d))
    mask = np.where(rng.random((sq, sk)) < 0.3, -1e30, 0.0)
    mask[:, 0] = 0.0
    out = O.attention(s, v, 0.5, mask=mask)
    for i in range(sq):
        w = np.exp(s[i] * 0.5 + mask[i] - np.max(s[i] * 0.5 + mask[i]))
        w /= w.sum()
        assert np.allclose(out[i], w @ v)
    causal = O.attention(s, v, 1.0, causal=True)
    for i in range(sq):
        lim = i + (sk - sq)
        w = np.exp(s[i, : lim + 1] - s[i, : lim + 1].max())
        w /= w.sum()
        assert np.allclose(causal[i], w @ v[: lim + 1])


def test_oracle_detects_planted_mistakes():
    """A dropped term, a wrong sign or a transposed operand must change the answer."""
    rng = np.random.default_rng(9)
    d = 8
    pi = _orth(d, 3)
    s = rng.standard_normal((d, d)).astype(np.float32)
    cent = np.array([-0.4, -0.1, 0.1, 0.4], np.float32)
    bounds = (cent[:-1] + cent[1:]) / 2
    x = rng.standard_normal((4, d)).astype(np.float32)
    good = O.key_compress_packed(x, pi, s, cent, bounds, 2)
    bad_t = O.key_compress_packed(x, pi.T.copy(), s, cent, bounds, 2)
    assert not np.array_equal(good["packed_key_indices"], bad_t["packed_key_indices"])
    bad_s = O.key_compress_packed(x, pi, s.T.copy(), cent, bounds, 2)
    assert not np.array_equal(good["packed_qjl_signs"], bad_s["packed_qjl_signs"])
