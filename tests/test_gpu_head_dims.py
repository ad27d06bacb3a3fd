"""GPU parity at head dims other than 32 / 64 / 128 / 256.

The reference accepts any head_dim (kernels/attention.py:158-194 loops over d and
m, bit_ops.py:162-164 sizes packed rows for any d, compressors.py:42-70 builds
Pi and S for any d).  The HIP path takes every multiple of 8 up to 256: the
tile kernels pad the MFMA tiles to a multiple of 32 with zeros and read / write
packed rows of d*b/8 bytes, which are not dword aligned in general (d = 80 has
10-byte sign rows).  Bars as in test_gpu_kernels.py: codes and signs bit-exact
given the device's f32 decision inputs, norms within one f16 ulp, scores and
attention within rel-err 1e-3 and cosine 0.9999 of the float64 oracle on the
device's planes.
"""

import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from turboquant_pytorch import compressed_attention
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL = 1e-3
DIMS = [40, 80, 96, 112, 160, 192, 200]


def _case(**kw):
    print("case:", kw, flush=True)


def _np(t):
    return t.detach().cpu().numpy()


def _f16_ulps(a, b):
    a = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    b = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    return np.abs(a - b)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("d", DIMS)
def test_compress_keys_any_dim(d, bits):
    _case(d=d, bits=bits)
    torch.manual_seed(d * 10 + bits)
    x = torch.randn(2, 3, 37, d).to(torch.bfloat16)
    x[..., :4] *= 20.0
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    n = 2 * 3 * 37
    y_dev = torch.empty(n, d, device=DEV)
    p_dev = torch.empty(n, d, device=DEV)
    ck = kc._compress_gpu(x.to(DEV), y_out=y_dev, proj_out=p_dev)
    y_dev, p_dev = _np(y_dev), _np(p_dev)
    xs = x.float().numpy()
    ref = O.key_compress_packed(xs, kc.Pi.cpu().numpy(), kc.S.cpu().numpy(), kc.centroids.cpu().numpy(),
                                kc.boundaries.cpu().numpy(), kc.mse_bits, y=y_dev)
    assert ck["packed_key_indices"].shape == (n, O.out_cols(d, bits - 1))
    assert ck["packed_qjl_signs"].shape == (n, d // 8)
    assert np.array_equal(_np(ck["packed_key_indices"]), ref["packed_key_indices"])
    assert np.array_equal(_np(ck["packed_qjl_signs"]), O.pack_bits((p_dev >= 0).astype(np.int32), 1))
    own = O.rotate(xs, kc.Pi.cpu().numpy())[2]
    assert np.max(np.abs(y_dev - own)) < 2e-6
    assert O.rel_err(p_dev, ref["proj"]) < 1e-5
    assert _f16_ulps(_np(ck["vec_norms"]).reshape(-1), ref["vec_norms"]).max() <= 1
    assert _f16_ulps(_np(ck["residual_norm"]).reshape(-1), ref["residual_norm"]).max() <= 1


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("d", DIMS)
def test_compress_values_and_decompress_any_dim(d, bits):
    _case(d=d, bits=bits)
    torch.manual_seed(7 * d + bits)
    x = torch.randn(1, 5, 29, d).to(torch.bfloat16)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    n = 5 * 29
    y_dev = torch.empty(n, d, device=DEV)
    cv = vc._compress_gpu(x.to(DEV), y_out=y_dev)
    y_dev = _np(y_dev)
    xs = x.float().numpy()
    ref = O.value_compress_packed(xs, vc.Pi.cpu().numpy(), vc.boundaries.cpu().numpy(), bits, y=y_dev)
    assert cv["packed_indices"].shape == (n, O.out_cols(d, bits))
    assert np.array_equal(_np(cv["packed_indices"]), ref["packed_indices"])
    assert _f16_ulps(_np(cv["vec_norms"]), ref["vec_norms"]).max() <= 1
    assert np.max(np.abs(y_dev - O.rotate(xs, vc.Pi.cpu().numpy())[2])) < 2e-6
    rec = _np(vc.decompress(cv)).reshape(n, d)
    rref = O.value_decompress(ref["codes"], _np(cv["vec_norms"]), vc.Pi.cpu().numpy(), vc.centroids.cpu().numpy())
    assert O.rel_err(rec, rref) < 1e-5


@pytest.mark.parametrize("d", DIMS)
def test_query_prep_any_dim(d):
    _case(d=d)
    torch.manual_seed(d)
    q = torch.randn(2, 4, 21, d, device=DEV, dtype=torch.bfloat16) * 3
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    q_rot, q_proj = kc.prepare_queries(q)
    assert q_rot.shape == (2, 4, 21, d) and q_proj.shape == (2, 4, 21, d)
    qs = q.float().cpu().numpy().reshape(-1, d).astype(np.float64)
    pi = kc.Pi.cpu().numpy().astype(np.float64)
    exact = qs @ pi.T
    got = _np(q_rot).reshape(-1, d).astype(np.float64)
    # f16 rounding of an f32-grade dot product (half an f16 ulp + the dot-product bound)
    excess = (np.abs(got - exact) - (2.0 ** -11 * np.abs(exact) + 2.0 ** -25)) / (np.abs(qs) @ np.abs(pi).T)
    assert excess.max() <= 2.0 ** -17
    se16 = _np(kc._dev_tables.s_eff16).astype(np.float64)
    proj_ref = got @ se16.T
    got_p = _np(q_proj).reshape(-1, d).astype(np.float64)
    assert np.all(np.abs(got_p - proj_ref) <= 2.0 ** -24 * np.abs(proj_ref) + 2.0 ** -17 * (np.abs(got) @ np.abs(se16).T))


def _planes(ck, d, mse_bits):
    codes = O.unpack_bits(_np(ck["packed_key_indices"]), mse_bits, d)
    signs = O.unpack_bits(_np(ck["packed_qjl_signs"]), 1, d)
    return codes, signs, _np(ck["residual_norm"]).reshape(-1), _np(ck["vec_norms"]).reshape(-1)


def _oracle_scores(kc, q, ck, hq, hkv):
    B, _, Sq, d = q.shape
    Sk = ck["shape"][2]
    codes, signs, rn, vn = _planes(ck, d, kc.mse_bits)
    q_rot, q_proj = O.query_prep(q.float().cpu().numpy(), kc.Pi.cpu().numpy(), kc._dev_tables.s_eff16.cpu().numpy())
    q_rot, q_proj = q_rot.reshape(B, hq, Sq, d), q_proj.reshape(B, hq, Sq, d)
    g = hq // hkv
    out = np.zeros((B, hq, Sq, Sk))
    for b in range(B):
        for h in range(hq):
            r = slice((b * hkv + h // g) * Sk, (b * hkv + h // g + 1) * Sk)
            out[b, h] = O.scores_packed(q_rot[b, h], q_proj[b, h], codes[r], signs[r], rn[r], vn[r],
                                        kc.centroids.cpu().numpy().astype(np.float16), O.COEFF(d))
    return out


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("d", DIMS)
def test_scores_any_dim(d, bits):
    # Sk = 77 leaves a partial last tile; odd Sk puts tiles at every byte alignment of 10-byte rows
    _case(d=d, bits=bits)
    torch.manual_seed(d + bits)
    hq, hkv, sq, sk = 8, 2, 5, 77
    k = torch.randn(2, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    q = torch.randn(2, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    ck = kc.compress(k)
    got = _np(kc.asymmetric_attention_scores(q, ck))
    ref = _oracle_scores(kc, q, ck, hq, hkv)
    assert got.shape == ref.shape
    assert O.rel_err(got, ref) < REL


def _oracle_attention(kc, vc, q, ck, cv, hq, hkv, mask=None, causal=False):
    B, _, Sq, d = q.shape
    Sk = ck["shape"][2]
    scores = _oracle_scores(kc, q, ck, hq, hkv)
    codes_v = O.unpack_bits(_np(cv["packed_indices"]), vc.bits, d)
    vals = O.value_decompress(codes_v, _np(cv["vec_norms"]), vc.Pi.cpu().numpy(), vc.centroids.cpu().numpy())
    vals = vals.reshape(B, hkv, Sk, d)
    g = hq // hkv
    out = np.zeros((B, Sq, hq, d))
    for b in range(B):
        for h in range(hq):
            m = None if mask is None else np.broadcast_to(mask, (B, hq, Sq, Sk))[b, h]
            out[b, :, h] = O.attention(scores[b, h], vals[b, h // g], 1 / math.sqrt(d), mask=m, causal=causal)
    return out


@pytest.mark.parametrize("bits,hq,hkv,sq,sk,causal", [
    (3, 8, 2, 45, 45, True), (2, 4, 4, 1, 133, False), (4, 16, 2, 19, 70, True),
])
@pytest.mark.parametrize("d", DIMS)
def test_attention_any_dim(d, bits, hq, hkv, sq, sk, causal):
    _case(d=d, bits=bits, hq=hq, hkv=hkv, sq=sq, sk=sk, causal=causal)
    torch.manual_seed(sq + 7 * sk + d)
    q = torch.randn(2, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(2, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(2, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    got = _np(compressed_attention(q, kc, vc, ck, cv, causal=causal, out_dtype=torch.float32))
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, causal=causal)
    assert got.shape == ref.shape
    assert O.rel_err(got, ref) < REL and O.cosine(got, ref) > 0.9999


@pytest.mark.parametrize("d", [80, 112, 192])
def test_attention_mask_and_output_dtypes_any_dim(d):
    _case(d=d)
    torch.manual_seed(11 + d)
    B, hq, hkv, S = 2, 4, 2, 45
    q = torch.randn(B, hq, S, d, device=DEV)
    k = torch.randn(B, hkv, S, d, device=DEV)
    v = torch.randn(B, hkv, S, d, device=DEV)
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, 3, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    mask = torch.zeros(B, 1, S, S)
    mask[0, 0, :, :33] = torch.finfo(torch.float32).min  # left padding on batch 0
    mask[0, 0, :33, :] = 0.0  # rows with no real key keep uniform weights over their own
    mask = mask + torch.triu(torch.full((S, S), torch.finfo(torch.float32).min), 1)
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, mask=mask.numpy())
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        got = compressed_attention(q, kc, vc, ck, cv, attention_mask=mask.to(DEV), out_dtype=dt)
        assert got.dtype == dt and got.shape == (B, S, hq, d)
        tol = REL if dt == torch.float32 else 1e-2
        assert O.rel_err(_np(got.float()), ref) < tol


def test_unsupported_head_dim_raises():
    _case(what="d=100")
    kc = TurboQuantCompressorV2(100, 3, seed=42, device=DEV)
    with pytest.raises(RuntimeError, match="100"):
        kc.compress(torch.randn(1, 1, 4, 100, device=DEV))


@pytest.mark.parametrize("d,bits,vbits,hq,hkv,sq,sk,causal,masked", [
    (64, 3, 3, 32, 8, 1, 5000, False, False),    # Llama-3.2-1B-shaped decode step
    (64, 2, 2, 12, 12, 1, 9000, False, True),    # GPT-2-shaped decode, padding mask
    (64, 4, 4, 16, 2, 2, 3000, True, False),     # two query rows, causal
    (80, 3, 3, 8, 2, 1, 4000, False, False),     # 10-byte sign rows (byte-stream staging)
    (96, 2, 2, 4, 4, 3, 2500, True, False),
    (256, 3, 3, 8, 2, 1, 3000, False, False),    # partial rows of 256 floats
    (40, 3, 3, 4, 1, 1, 2100, False, False),     # head dim padded to 64
    (128, 3, 2, 32, 8, 1, 6000, False, False),   # value bits below the key bits (no decode kernels)
    (128, 3, 3, 64, 2, 1, 4000, False, False),   # 32 columns per kv head (beyond the decode kernels)
])
def test_attention_split_keys_any_dim(d, bits, vbits, hq, hkv, sq, sk, causal, masked):
    """The tiled kernel split over keys (few query rows per kv head, long key ranges) and its
    merge, against the float64 oracle and against the unsplit tiled kernel."""
    _case(d=d, bits=bits, vbits=vbits, hq=hq, hkv=hkv, sq=sq, sk=sk, causal=causal, masked=masked)
    from turboquant_pytorch import _native
    B = 2
    assert _native.lib().tq_attention_workspace_size(B, hq, hkv, sq, sk, d, bits) > 0
    torch.manual_seed(d + 3 * sk + sq)
    q = torch.randn(B, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, vbits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    mask = None
    if masked:
        mask = torch.zeros(B, 1, sq, sk)
        mask[0, 0, :, : sk // 4] = torch.finfo(torch.float32).min  # left padding on batch row 0
        mask[1, 0, :, 11] = -2.5
    mdev = mask.to(DEV) if mask is not None else None
    got = _np(compressed_attention(q, kc, vc, ck, cv, attention_mask=mdev, causal=causal, out_dtype=torch.float32))
    unsplit = _np(compressed_attention(q, kc, vc, ck, cv, attention_mask=mdev, causal=causal,
                                       out_dtype=torch.float32, split_k=False))
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, mask=mask.numpy() if mask is not None else None,
                            causal=causal)
    err, err_u = O.rel_err(got, ref), O.rel_err(unsplit, ref)
    print(f"split rel-err {err:.2e}, unsplit {err_u:.2e}", flush=True)
    assert np.isfinite(got).all()
    assert err < REL and O.cosine(got, ref) > 0.9999
    assert err_u < REL


@pytest.mark.parametrize("d,bits,hq,hkv,sq,sk", [
    (64, 3, 32, 8, 1, 5001),    # blocks split the keys; the last split ends inside a tile
    (80, 2, 12, 12, 1, 3000),   # byte-stream rows
    (256, 4, 8, 2, 2, 2600),
    (128, 3, 64, 2, 1, 3000),   # 32 columns per kv head (beyond the decode kernels)
])
def test_scores_split_keys_any_dim(d, bits, hq, hkv, sq, sk):
    """Materialised scores of few-query shapes over long key ranges, with the keys split over
    blocks, against the float64 oracle."""
    _case(d=d, bits=bits, hq=hq, hkv=hkv, sq=sq, sk=sk)
    torch.manual_seed(d + bits + sk)
    k = torch.randn(2, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    q = torch.randn(2, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    ck = kc.compress(k)
    got = _np(kc.asymmetric_attention_scores(q, ck))
    ref = _oracle_scores(kc, q, ck, hq, hkv)
    assert got.shape == ref.shape and np.isfinite(got).all()
    assert O.rel_err(got, ref) < REL
