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


# ---------------------------------------------------------------- packed estimator == unpacked estimator
#
# The packed scorer (attention.py:419-461, with q_rot and S_eff from compressors.py:186-189)
# and the unpacked scorer (compressors.py:201-224, pinned by the reference's golden vectors
# in tests/golden/cpu_compress.npz) are two forms of one estimator:
#   vn <q Pi^T, C[c]>          = <q, (C[c] Pi) vn>          = <q, k_mse>
#   <q Pi^T (S Pi^T)^T, s>     = <q Pi^T Pi S^T, s>          = <q S^T, s>
# so on planes of the same key compression they must agree to rounding.  Each check
# below is evaluated with the oracle functions and then with planted mistakes, which
# must fail it: Pi <-> Pi^T, S_eff <-> S_eff^T, vn <-> rn, a {0,1} sign used where
# 2*bit-1 belongs, a reversed codebook, a dropped QJL term.

def _exact_orthogonal(d, seed):
    q, r = np.linalg.qr(np.random.default_rng(seed).standard_normal((d, d)))
    return q * np.sign(np.diag(r))[None, :]


def _f16_exact(rng, shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16).astype(np.float64)


def _packed_vs_unpacked_err(pi, s, cent, bounds, mse_bits, x, q, scores_fn=None, prep_fn=None,
                            exact_prep=False):
    """max |packed - unpacked| / max |unpacked| over one key set.

    The packed side gets q_rot = q Pi^T and q_proj = q_rot S_eff^T (float64, unrounded, or
    through prep_fn), S_eff = S Pi^T; the unpacked side gets q, k_mse = (C16[codes] Pi) vn
    and +-1 signs, with the codes, sign bits and norms of one packed compression."""
    scores_fn = scores_fn or O.scores_packed
    d = pi.shape[0]
    comp = O.key_compress_packed(x, pi.astype(np.float32), s.astype(np.float32), cent, bounds, mse_bits)
    codes = O.unpack_bits(comp["packed_key_indices"], mse_bits, d)
    sbits = O.unpack_bits(comp["packed_qjl_signs"], 1, d)
    rn = comp["residual_norm"].astype(np.float64)
    vn = comp["vec_norms"].astype(np.float64)
    c16 = np.asarray(cent, np.float32).astype(np.float16)
    s_eff = s @ pi.T
    if prep_fn is None:
        q_rot = q @ pi.T
        q_proj = q_rot @ s_eff.T
    else:
        q_rot, q_proj = prep_fn(q, pi, s_eff)
    packed = scores_fn(q_rot, q_proj, codes, sbits, rn, vn, c16, O.COEFF(d))
    k_mse = (c16.astype(np.float64)[codes] @ pi) * vn[:, None]
    unpacked = O.scores_unpacked(q, k_mse, sbits * 2.0 - 1.0, rn, s, O.COEFF(d))
    return float(np.max(np.abs(packed - unpacked)) / np.max(np.abs(unpacked)))


def _setup(d, bits, real):
    """(Pi, S, centroids, boundaries) as float64: the real compressor's (f32) matrices, or an
    exactly orthogonal float64 Pi with a Gaussian S."""
    from turboquant_pytorch.compressors import TurboQuantCompressorV2

    kc = TurboQuantCompressorV2(d, bits, seed=42)
    cent, bounds = kc.centroids.numpy(), kc.boundaries.numpy()
    if real:
        return kc.Pi.double().numpy(), kc.S.double().numpy(), cent, bounds, kc.mse_bits
    rng = np.random.default_rng(d + bits)
    return _exact_orthogonal(d, d * 7 + bits), rng.standard_normal((d, d)), cent, bounds, kc.mse_bits


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("d", [64, 128])
def test_packed_estimator_equals_unpacked(d, bits):
    rng = np.random.default_rng(100 + d + bits)
    x = rng.standard_normal((40, d)).astype(np.float32)
    x[:, :3] *= 20  # outlier channels, as in the benchmark keys
    q = rng.standard_normal((6, d)).astype(np.float32).astype(np.float64)  # scores_unpacked takes f32 q
    # exactly orthogonal Pi: the identity holds to float64 rounding
    assert _packed_vs_unpacked_err(*_setup(d, bits, real=False), x, q) < 1e-12
    # the compressor's own f32 Pi and S: Pi^T Pi = I to f32 rounding
    assert _packed_vs_unpacked_err(*_setup(d, bits, real=True), x, q) < 2e-6


def _mut_vn_rn(qr, qp, codes, sb, rn, vn, c16, coeff):
    return O.scores_packed(qr, qp, codes, sb, vn, rn, c16, coeff)


def _mut_sign01(qr, qp, codes, sb, rn, vn, c16, coeff):
    # 2*b' - 1 = b  <=>  the estimator uses the raw {0,1} bit where +-1 belongs
    return O.scores_packed(qr, qp, codes, (np.asarray(sb, np.float64) + 1) / 2, rn, vn, c16, coeff)


def _mut_codebook(qr, qp, codes, sb, rn, vn, c16, coeff):
    return O.scores_packed(qr, qp, codes, sb, rn, vn, c16[::-1].copy(), coeff)


def _mut_no_qjl(qr, qp, codes, sb, rn, vn, c16, coeff):
    return O.scores_packed(qr, qp, codes, sb, rn, vn, c16, 0.0)


@pytest.mark.parametrize("mutant", [_mut_vn_rn, _mut_sign01, _mut_codebook, _mut_no_qjl])
@pytest.mark.parametrize("real", [False, True])
def test_packed_estimator_identity_catches_planted_mistakes(mutant, real):
    d, bits = 64, 3
    rng = np.random.default_rng(7)
    x = rng.standard_normal((40, d)).astype(np.float32)
    q = rng.standard_normal((6, d)).astype(np.float32).astype(np.float64)
    assert _packed_vs_unpacked_err(*_setup(d, bits, real), x, q, scores_fn=mutant) > 1e-2


def _prep_exact(transpose_pi=False, transpose_seff=False):
    """q_rot, q_proj through O.query_prep on inputs whose f16 roundings are exact: q is built
    as q_rot16 Pi from f16 values and S_eff is itself f16, so every rounding the reference
    applies (compressors.py:186, :189) is the identity and float64 equality is expected."""

    def prep(q, pi, s_eff):
        s16 = s_eff.astype(np.float16)
        qr, qp = O.query_prep(q, pi.T if transpose_pi else pi, s16.T if transpose_seff else s16)
        return qr.astype(np.float64), qp

    return prep


@pytest.mark.parametrize("d", [64, 128])
def test_query_prep_identities(d):
    rng = np.random.default_rng(d)
    pi = _exact_orthogonal(d, 5 + d)
    s_eff16 = _f16_exact(rng, (d, d))
    s = s_eff16 @ pi  # so that f16(S Pi^T) = s_eff16 exactly
    qr16 = _f16_exact(rng, (8, d))
    q = qr16 @ pi  # so that f16(q Pi^T) = qr16 exactly
    q_rot, q_proj = O.query_prep(q, pi, s_eff16.astype(np.float16))
    # <q_rot, y> = <q, y Pi>: the rotated query scores rotated vectors as q scores the originals
    y = rng.standard_normal((5, d))
    assert np.max(np.abs(q_rot.astype(np.float64) @ y.T - q @ (y @ pi).T)) < 1e-10
    # q_proj = q S^T: the packed QJL projection equals the unpacked one
    assert np.max(np.abs(q_proj - q @ s.T)) < 1e-9 * np.max(np.abs(q @ s.T))
    # q_rot is the f16 rounding of q Pi^T (compressors.py:186)
    qr_gen = (rng.standard_normal((8, d))).astype(np.float32)
    r16, _ = O.query_prep(qr_gen, pi, s_eff16.astype(np.float16))
    assert np.array_equal(r16, (qr_gen.astype(np.float64) @ pi.T).astype(np.float32).astype(np.float16))


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_query_prep_composes_with_packed_estimator(bits):
    d = 128
    pi = _exact_orthogonal(d, 31)
    rng = np.random.default_rng(bits)
    s = _f16_exact(rng, (d, d)) @ pi
    from turboquant_pytorch.compressors import TurboQuantCompressorV2

    kc = TurboQuantCompressorV2(d, bits, seed=42)
    x = rng.standard_normal((32, d)).astype(np.float32)
    q = _f16_exact(rng, (4, d)) @ pi
    args = (pi, s, kc.centroids.numpy(), kc.boundaries.numpy(), kc.mse_bits, x, q)
    # scores_unpacked rounds q to f32 (the reference's .float()), hence 1e-6 and not 1e-12
    assert _packed_vs_unpacked_err(*args, prep_fn=_prep_exact()) < 1e-6
    assert _packed_vs_unpacked_err(*args, prep_fn=_prep_exact(transpose_pi=True)) > 1e-2
    assert _packed_vs_unpacked_err(*args, prep_fn=_prep_exact(transpose_seff=True)) > 1e-2
