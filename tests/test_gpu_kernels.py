"""GPU parity of the gfx950 kernels against the CPU oracle.

Bars (from the task contract): packed codes, sign bits and centroid indices are
bit-exact given the same f32 rotated rows / projections (the kernels report the
f32 values they decided on through y_out / proj_out); scores and attention
outputs are within rel-err 1e-3 (or cosine >= 0.9999) of the float64 oracle
estimator evaluated on the same packed planes.
"""

import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from turboquant_pytorch import compressed_attention
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2
from turboquant_pytorch.kernels import (asymmetric_attention_scores, lloyd_max_dequantize,
                                        lloyd_max_quantize, pack_bits, unpack_bits)

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL = 1e-3


def _case(**kw):
    print("case:", kw, flush=True)


def _np(t):
    return t.detach().cpu().numpy()


def _f16_ulps(a, b):
    a = np.asarray(a, np.float16).view(np.int16).astype(np.int32)
    b = np.asarray(b, np.float16).view(np.int16).astype(np.int32)
    return np.abs(a - b)


# ---------------------------------------------------------------- bit ops

@pytest.mark.parametrize("b", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("d", [7, 128])
def test_pack_unpack(b, d):
    _case(b=b, d=d)
    torch.manual_seed(99 + b)
    idx = torch.randint(0, 1 << b, (100, d), dtype=torch.int32)
    packed = pack_bits(idx.to(DEV), b)
    assert np.array_equal(_np(packed), O.pack_bits(idx.numpy(), b))
    assert torch.equal(unpack_bits(packed, b, d).cpu(), idx)
    # codes are masked to b bits (bit_ops.py:274)
    wide = idx + (1 << b)
    assert torch.equal(pack_bits(wide.to(DEV), b).cpu(), packed.cpu())


@pytest.mark.parametrize("b_eff", [1, 2, 3, 4])
def test_quantize_bit_exact_including_boundaries(b_eff):
    _case(b_eff=b_eff)
    vc = TurboQuantCompressorMSE(128, b_eff, seed=0)
    bounds = vc.boundaries.numpy()
    rng = np.random.default_rng(13)
    y = (rng.standard_normal((100, 128)) / math.sqrt(128)).astype(np.float32)
    # plant exact boundaries and +-1 ulp neighbours
    flat = y.reshape(-1)
    k = 0
    for bv in bounds:
        for v in (np.nextafter(bv, -np.inf), bv, np.nextafter(bv, np.inf)):
            flat[k] = v
            k += 1
    packed = lloyd_max_quantize(torch.from_numpy(y).to(DEV), vc.boundaries.to(DEV), b_eff)
    assert np.array_equal(_np(packed), O.pack_bits(O.quantize_searchsorted(y, bounds), b_eff))
    deq = lloyd_max_dequantize(packed, vc.centroids.half().to(DEV), b_eff, 128)
    assert deq.dtype == torch.float16
    assert np.array_equal(_np(deq), O.dequantize(_np(packed), vc.centroids.numpy(), b_eff, 128))


# ---------------------------------------------------------------- compression

DTYPES = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("d", [32, 64, 128, 256])
def test_compress_keys(d, bits, dt):
    _case(d=d, bits=bits, dt=dt)
    torch.manual_seed(d + bits)
    x = torch.randn(2, 3, 37, d).to(DTYPES[dt])
    x[..., :4] *= 20.0  # outlier channels as in the config-2 workload
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    n = x[0].numel() * 2 // d
    y_dev = torch.empty(n, d, device=DEV)
    p_dev = torch.empty(n, d, device=DEV)
    ck = kc._compress_gpu(x.to(DEV), y_out=y_dev, proj_out=p_dev)
    y_dev, p_dev = _np(y_dev), _np(p_dev)
    xs = x.float().numpy()
    ref = O.key_compress_packed(xs, kc.Pi.cpu().numpy(), kc.S.cpu().numpy(), kc.centroids.cpu().numpy(),
                                kc.boundaries.cpu().numpy(), kc.mse_bits, y=y_dev)
    # stage-wise bit exactness
    assert np.array_equal(_np(ck["packed_key_indices"]), ref["packed_key_indices"])
    assert np.array_equal(_np(ck["packed_qjl_signs"]), O.pack_bits((p_dev >= 0).astype(np.int32), 1))
    # the f32 decision inputs agree with the oracle's f32 computation
    own = O.rotate(xs, kc.Pi.cpu().numpy())[2]
    assert np.max(np.abs(y_dev - own)) < 2e-6
    assert O.rel_err(p_dev, ref["proj"]) < 1e-5
    assert np.mean(O.quantize_searchsorted(own, kc.boundaries.cpu().numpy()) != ref["codes"]) < 1e-3
    assert _f16_ulps(_np(ck["vec_norms"]).reshape(-1), ref["vec_norms"]).max() <= 1
    assert _f16_ulps(_np(ck["residual_norm"]).reshape(-1), ref["residual_norm"]).max() <= 1
    assert ck["residual_norm"].shape == (2, 3, 37) and ck["packed_qjl_signs"].shape == (n, d // 8)


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
@pytest.mark.parametrize("d", [64, 128])
def test_compress_values_and_decompress(d, bits, dt):
    _case(d=d, bits=bits, dt=dt)
    torch.manual_seed(7 * d + bits)
    x = torch.randn(1, 5, 29, d).to(DTYPES[dt])
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    n = 5 * 29
    y_dev = torch.empty(n, d, device=DEV)
    cv = vc._compress_gpu(x.to(DEV), y_out=y_dev)
    y_dev = _np(y_dev)
    xs = x.float().numpy()
    ref = O.value_compress_packed(xs, vc.Pi.cpu().numpy(), vc.boundaries.cpu().numpy(), bits, y=y_dev)
    assert np.array_equal(_np(cv["packed_indices"]), ref["packed_indices"])
    assert _f16_ulps(_np(cv["vec_norms"]), ref["vec_norms"]).max() <= 1
    own = O.rotate(xs, vc.Pi.cpu().numpy())[2]
    assert np.max(np.abs(y_dev - own)) < 2e-6
    rec = _np(vc.decompress(cv)).reshape(n, d)
    rref = O.value_decompress(ref["codes"], _np(cv["vec_norms"]), vc.Pi.cpu().numpy(), vc.centroids.cpu().numpy())
    assert O.rel_err(rec, rref) < 1e-5


def test_compress_strided_views_match_contiguous():
    _case(what="strided")
    torch.manual_seed(3)
    base = torch.randn(2, 40, 4, 128, device=DEV, dtype=torch.bfloat16)  # [B, T, H, D]
    view = base.transpose(1, 2)  # [B, H, T, D] non-contiguous, as the families produce
    kc = TurboQuantCompressorV2(128, 3, seed=1, device=DEV)
    a, b = kc.compress(view), kc.compress(view.contiguous())
    for k in ("packed_key_indices", "packed_qjl_signs", "residual_norm", "vec_norms"):
        assert torch.equal(a[k], b[k]), k


# ---------------------------------------------------------------- scoring

def _planes(ck, d, mse_bits):
    codes = O.unpack_bits(_np(ck["packed_key_indices"]), mse_bits, d)
    signs = O.unpack_bits(_np(ck["packed_qjl_signs"]), 1, d)
    return codes, signs, _np(ck["residual_norm"]).reshape(-1), _np(ck["vec_norms"]).reshape(-1)


def _oracle_scores(kc, q, ck, hq, hkv):
    """float64 oracle scores [B, Hq, Sq, Sk] from the device's planes."""
    B, _, Sq, d = q.shape
    Sk = ck["shape"][2]
    codes, signs, rn, vn = _planes(ck, d, kc.mse_bits)
    q_rot, q_proj = O.query_prep(q.float().cpu().numpy(), kc.Pi.cpu().numpy(),
                                 kc._dev_tables.s_eff16.cpu().numpy())
    q_rot = q_rot.reshape(B, hq, Sq, d)
    q_proj = q_proj.reshape(B, hq, Sq, d)
    g = hq // hkv
    out = np.zeros((B, hq, Sq, Sk))
    for b in range(B):
        for h in range(hq):
            r = slice((b * hkv + h // g) * Sk, (b * hkv + h // g + 1) * Sk)
            out[b, h] = O.scores_packed(q_rot[b, h], q_proj[b, h], codes[r], signs[r], rn[r], vn[r],
                                        kc.centroids.cpu().numpy().astype(np.float16), O.COEFF(d))
    return out


@pytest.mark.parametrize("d,bits,hq,hkv,sq,sk", [
    (128, 3, 8, 2, 5, 77), (128, 2, 4, 4, 1, 1), (128, 4, 32, 8, 3, 130),
    (64, 3, 12, 12, 33, 65), (32, 2, 2, 1, 9, 64), (256, 3, 4, 2, 17, 40),
])
def test_scores_match_oracle(d, bits, hq, hkv, sq, sk):
    _case(d=d, bits=bits, hq=hq, hkv=hkv, sq=sq, sk=sk)
    torch.manual_seed(sq * 131 + sk)
    k = torch.randn(2, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    q = torch.randn(2, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    ck = kc.compress(k)
    got = _np(kc.asymmetric_attention_scores(q, ck))
    ref = _oracle_scores(kc, q, ck, hq, hkv)
    assert got.shape == ref.shape
    assert O.rel_err(got, ref) < REL


def test_query_prep_matches_oracle():
    _case(what="query_prep")
    torch.manual_seed(5)
    q = torch.randn(2, 8, 50, 128, device=DEV, dtype=torch.bfloat16) * 3
    kc = TurboQuantCompressorV2(128, 3, seed=42, device=DEV)
    q_rot, q_proj = kc.prepare_queries(q)
    rot_ref, _ = O.query_prep(q.float().cpu().numpy(), kc.Pi.cpu().numpy(), kc._dev_tables.s_eff16.cpu().numpy())
    exact = q.float().cpu().numpy().reshape(-1, 128).astype(np.float64) @ kc.Pi.cpu().numpy().astype(np.float64).T
    got = _np(q_rot).reshape(-1, 128).astype(np.float64)
    # f16 rounding of an f32-grade dot product: each element lies within half an
    # f16 ulp plus the standard dot-product bound 2^-17 * sum_j |q_j Pi_ij|
    # (n * u for n = 128, u = 2^-24) of the exact value, and rounds like the
    # oracle's f32 GEMM almost everywhere
    absum = np.abs(q.float().cpu().numpy().reshape(-1, 128).astype(np.float64)) @ np.abs(kc.Pi.cpu().numpy().astype(np.float64)).T
    half_ulp = 2.0 ** -11 * np.abs(exact) + 2.0 ** -25  # f16 rounding bound u|x| (+ subnormal step)
    excess = (np.abs(got - exact) - half_ulp) / absum
    print(f"q_rot: rel-err {O.rel_err(got, exact):.2e}, worst excess/absum {excess.max():.2e}, "
          f"mismatch vs oracle {(got != rot_ref).mean():.2e}")
    assert O.rel_err(got, exact) < 5e-4
    assert excess.max() <= 2.0 ** -17
    assert (got != rot_ref).mean() < 0.01
    # q_proj: f32, the f32 accumulation of exact f16 products (kernels/attention.py:158-167, :453):
    # within the dot-product bound 2^-17 * sum |q_rot_j S_eff_ij| of the exact value
    assert q_proj.dtype == torch.float32
    qr16 = _np(q_rot).reshape(-1, 128).astype(np.float64)
    se16 = _np(kc._dev_tables.s_eff16).astype(np.float64)
    proj_ref = qr16 @ se16.T
    proj_abs = np.abs(qr16) @ np.abs(se16).T
    got_p = _np(q_proj).reshape(-1, 128).astype(np.float64)
    assert np.all(np.abs(got_p - proj_ref) <= 2.0 ** -24 * np.abs(proj_ref) + 2.0 ** -17 * proj_abs)
    print(f"q_proj: worst |err| / sum|terms| {np.max(np.abs(got_p - proj_ref) / proj_abs):.2e}")


def test_reference_kernel_api_gpu_matches_cpu():
    """kernels.asymmetric_attention_scores on GPU vs its CPU path (reference test_kernels.py:404-422)."""
    _case(what="kernel api")
    rng = np.random.default_rng(4)
    B, H, Sq, Sk, d, bits = 2, 4, 8, 16, 64, 3
    cent = torch.tensor([-0.2, -0.07, 0.07, 0.2]).half().unsqueeze(0).expand(H, -1).contiguous()
    args = dict(
        query=torch.from_numpy(rng.standard_normal((B, H, Sq, d))).half(),
        packed_key_indices=torch.from_numpy(O.pack_bits(rng.integers(0, 4, (B * H * Sk, d)), 2)).view(B, H, Sk, -1),
        packed_qjl_signs=torch.from_numpy(O.pack_bits(rng.integers(0, 2, (B * H * Sk, d)), 1)).view(B, H, Sk, -1),
        residual_norms=torch.from_numpy(rng.random((B, H, Sk))).half(),
        centroids=cent, qjl_matrix=torch.from_numpy(rng.standard_normal((d, d))).half(),
        vec_norms=torch.from_numpy(rng.random((B, H, Sk)) * 8).half(), b=bits, coeff=O.COEFF(d))
    cpu = asymmetric_attention_scores(**args)
    gpu = asymmetric_attention_scores(**{k: (v.to(DEV) if torch.is_tensor(v) else v) for k, v in args.items()})
    assert O.rel_err(_np(gpu), _np(cpu)) < REL
    assert (gpu.cpu() - cpu).abs().max().item() < 3e-2


@pytest.mark.parametrize("d,m,per_head", [(128, 64, False), (128, 96, True), (128, 200, False),
                                          (128, 256, False), (64, 100, True), (64, 20, False)])
def test_reference_kernel_api_gpu_non_square_qjl(d, m, per_head):
    """kernels.asymmetric_attention_scores on GPU with a QJL matrix of m != d rows (reference
    attention.py:274-300 takes qjl_matrix [m, d] and m-bit sign rows), against the float64
    oracle estimator on the same packed planes."""
    _case(what="kernel api, non-square QJL", d=d, m=m, per_head=per_head)
    rng = np.random.default_rng(d + m)
    B, H, Sq, Sk, bits = 2, 4, 3, 300, 3
    codes = rng.integers(0, 4, (B * H * Sk, d))
    sb = rng.integers(0, 2, (B * H * Sk, m))
    base = np.array([-0.2, -0.07, 0.07, 0.2])
    cent = np.stack([base * (1.0 + 0.1 * h if per_head else 1.0) for h in range(H)]).astype(np.float16)
    q = rng.standard_normal((B, H, Sq, d)).astype(np.float16)
    s_eff = rng.standard_normal((m, d)).astype(np.float16)
    rn = rng.random((B, H, Sk)).astype(np.float16)
    vn = (rng.random((B, H, Sk)) * 8).astype(np.float16)
    coeff = O.COEFF(d)
    got = _np(asymmetric_attention_scores(
        torch.from_numpy(q).to(DEV), torch.from_numpy(O.pack_bits(codes, 2)).view(B, H, Sk, -1).to(DEV),
        torch.from_numpy(O.pack_bits(sb, 1)).view(B, H, Sk, -1).to(DEV), torch.from_numpy(rn).to(DEV),
        torch.from_numpy(cent).to(DEV), torch.from_numpy(s_eff).to(DEV), torch.from_numpy(vn).to(DEV), bits, coeff))
    assert got.shape == (B, H, Sq, Sk)
    for bh in range(B * H):
        b_, h_ = divmod(bh, H)
        qp = q[b_, h_].astype(np.float64) @ s_eff.astype(np.float64).T
        ref = O.scores_packed(q[b_, h_], qp, codes[bh * Sk:(bh + 1) * Sk], sb[bh * Sk:(bh + 1) * Sk],
                              rn[b_, h_], vn[b_, h_], cent[h_], coeff)
        assert O.rel_err(got[b_, h_], ref) < REL, (bh, O.rel_err(got[b_, h_], ref))


# ---------------------------------------------------------------- fused attention

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


@pytest.mark.parametrize("d,bits,hq,hkv,sq,sk,causal", [
    (128, 3, 32, 8, 70, 70, True), (128, 3, 8, 2, 1, 300, False), (128, 2, 4, 4, 64, 64, True),
    (128, 4, 16, 2, 33, 97, True), (64, 3, 12, 12, 40, 40, False), (32, 3, 4, 2, 20, 20, True),
    (256, 3, 4, 4, 24, 50, True),
    # head_dim-128 prefill kernel: GQA groups that leave columns of a block unused (G=3) or give
    # 16 query rows per block (G=8), MHA non-causal with Sk > Sq, several causal blocks at bits 2 and 4
    (128, 2, 12, 4, 50, 50, True), (128, 3, 32, 4, 20, 300, True), (128, 4, 8, 8, 40, 90, False),
    (128, 2, 4, 2, 130, 130, True), (128, 4, 8, 2, 97, 160, True),
])
def test_attention_matches_oracle(d, bits, hq, hkv, sq, sk, causal):
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


@pytest.mark.parametrize("d", [64, 128])
def test_attention_additive_mask_and_dtypes(d):
    _case(what="mask", d=d)
    torch.manual_seed(11)
    B, hq, hkv, S = 2, 4, 2, 45
    q = torch.randn(B, hq, S, d, device=DEV)
    k = torch.randn(B, hkv, S, d, device=DEV)
    v = torch.randn(B, hkv, S, d, device=DEV)
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, 3, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    mask = torch.zeros(B, 1, S, S)
    mask[0, 0, :, 30:] = torch.finfo(torch.float32).min  # padding-style mask on batch 0
    mask = mask + torch.triu(torch.full((S, S), torch.finfo(torch.float32).min), 1)
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, mask=mask.numpy())
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        got = compressed_attention(q.to(dt), kc, vc, ck, cv, attention_mask=mask.to(DEV), out_dtype=dt)
        tol = REL if dt == torch.float32 else 8e-3
        assert O.rel_err(_np(got.float()), ref) < tol


@pytest.mark.parametrize("layout", ["per_head", "broadcast"])
def test_attention_additive_mask_vector_loads(layout):
    """d = 128 with key counts that are multiples of 4 and 16-byte aligned mask rows: the prefill
    kernel's masked form reads each lane's 4 consecutive mask values as one 16-byte load. Real
    bias values (ALiBi-like slopes, per head) on top of causal and padding masks, and a mask
    broadcast over batch and heads (zero strides), against the float64 oracle."""
    _case(what=f"mask vector loads {layout}")
    torch.manual_seed(12)
    B, hq, hkv, S, d = 2, 8, 2, 160, 128
    q = torch.randn(B, hq, S, d, device=DEV)
    k = torch.randn(B, hkv, S, d, device=DEV)
    v = torch.randn(B, hkv, S, d, device=DEV)
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, 3, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    causal = torch.triu(torch.full((S, S), torch.finfo(torch.float32).min), 1)
    if layout == "per_head":
        pos = torch.arange(S, dtype=torch.float32)
        slopes = torch.tensor([2.0 ** (-(h + 1)) for h in range(hq)])
        mask = -(slopes[None, :, None, None] * (pos[:, None] - pos[None, :]).abs()[None, None]).expand(B, hq, S, S).clone()
        mask[1, :, :, 100:] = torch.finfo(torch.float32).min  # padding on batch 1
        mask = mask + causal
    else:
        mask = (causal + 0.25 * torch.randn(S, S))[None, None]
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, mask=mask.numpy())
    got = compressed_attention(q, kc, vc, ck, cv, attention_mask=mask.to(DEV), out_dtype=torch.float32)
    assert O.rel_err(_np(got.float()), ref) < REL


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("npad", [40, 64, 100])
def test_attention_left_padding_mask(bits, npad):
    """An eager-style mask (causal plus left padding, both finfo.min) with `npad` padded keys on
    batch row 0: the first one to three 32-key tiles of every real query's column are fully
    masked before its first real key.  The padded query rows see only masked keys, which the
    reference's softmax of equal scores weighs equally.  Through the prefill kernel's
    additive-mask form (head_dim 128) against the float64 oracle, per batch row."""
    _case(what="left padding prefill", bits=bits, npad=npad)
    torch.manual_seed(5 * bits + npad)
    B, hq, hkv, S, d = 2, 8, 2, 200, 128
    q = torch.randn(B, hq, S, d, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(B, hkv, S, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, hkv, S, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    fmin = torch.finfo(torch.float32).min
    mask = torch.triu(torch.full((S, S), fmin), 1).expand(B, 1, S, S).clone()
    mask[0, 0, :, :npad] = fmin
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, mask=mask.numpy())
    got = _np(compressed_attention(q, kc, vc, ck, cv, attention_mask=mask.to(DEV), out_dtype=torch.float32))
    assert np.isfinite(got).all()
    for b in range(B):
        err = O.rel_err(got[b], ref[b])
        real = O.rel_err(got[b, npad:], ref[b, npad:])
        print(f"batch row {b}: rel-err {err:.2e} (real query rows {real:.2e})", flush=True)
        assert err < REL and real < REL, (b, err, real)


@pytest.mark.parametrize("bits,sq,sk,causal,masked", [
    (3, 160, 160, True, False),   # head_dim-128 prefill kernel, causal
    (2, 96, 224, False, False),   # prefill kernel, Sk > Sq
    (3, 160, 160, True, True),    # the prefill kernel's additive-mask form
    (3, 1, 2048, False, False),   # split-K decode kernels (bit-plane keys), 3 bits
    (2, 1, 2048, False, False),   # split-K decode kernels, 2 bits
])
def test_attention_rising_scores_rescale(bits, sq, sk, causal, masked):
    """Keys whose norms grow along the sequence (x1 to x9), so a column's scores climb by several
    times the lazy-rescale headroom (8 log2 units) over the keys: the rescale branch runs again and
    again, moving each column's reference and shifting the scores of the tile (held relative to
    the reference) before P = 2^(s - m). Against the float64 oracle."""
    _case(what="rising scores", bits=bits, sq=sq, sk=sk, causal=causal, masked=masked)
    torch.manual_seed(21 + sk + bits)
    B, hq, hkv, d = 2, 8, 2, 128
    q = 2.0 * torch.randn(B, hq, sq, d, device=DEV)
    ramp = 1.0 + 8.0 * torch.arange(sk, dtype=torch.float32) / sk
    k = torch.randn(B, hkv, sk, d) * ramp[None, None, :, None]
    k = k.to(DEV)
    v = torch.randn(B, hkv, sk, d, device=DEV)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    if masked:
        mask = torch.triu(torch.full((sq, sk), torch.finfo(torch.float32).min), 1 + sk - sq) + 0.5 * torch.randn(sq, sk)
        mask = mask[None, None]
        ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, mask=mask.numpy())
        got = compressed_attention(q, kc, vc, ck, cv, attention_mask=mask.to(DEV), out_dtype=torch.float32)
    else:
        ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, causal=causal)
        got = compressed_attention(q, kc, vc, ck, cv, causal=causal, out_dtype=torch.float32)
    got = _np(got.float())
    assert got.shape == ref.shape
    assert O.rel_err(got, ref) < REL and O.cosine(got, ref) > 0.9999


def test_attention_full_size_slice():
    """Config-2 shape (1 x 32 x 8192, 8 KV heads, bits=3), causal; oracle on a slice of query rows."""
    _case(what="config2 slice")
    torch.manual_seed(0)
    S, d = 8192, 128
    q = torch.randn(1, 32, S, d, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(1, 8, S, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(1, 8, S, d, device=DEV, dtype=torch.bfloat16)
    k[..., :4] *= 20
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, 3, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    out = compressed_attention(q, kc, vc, ck, cv, causal=True, out_dtype=torch.float32)
    assert torch.isfinite(out).all()
    rows = [0, 1, 63, 64, 4095, 8191]
    codes_v = O.unpack_bits(_np(cv["packed_indices"]), 3, d)
    vals = O.value_decompress(codes_v, _np(cv["vec_norms"]), vc.Pi.cpu().numpy(), vc.centroids.cpu().numpy())
    codes, signs, rn, vn = _planes(ck, d, kc.mse_bits)
    qs = q[:, :, rows]
    q_rot, q_proj = O.query_prep(qs.float().cpu().numpy(), kc.Pi.cpu().numpy(), kc._dev_tables.s_eff16.cpu().numpy())
    q_rot = q_rot.reshape(32, len(rows), d)
    q_proj = q_proj.reshape(32, len(rows), d)
    for h in (0, 5, 31):
        kv = h // 4
        r = slice(kv * S, (kv + 1) * S)
        sc = O.scores_packed(q_rot[h], q_proj[h], codes[r], signs[r], rn[r], vn[r],
                             kc.centroids.cpu().numpy().astype(np.float16), O.COEFF(d))
        for t, i in enumerate(rows):
            ref = O.attention(sc[t:t + 1, : i + 1], vals[r][: i + 1], 1 / math.sqrt(d))
            assert O.rel_err(_np(out[0, i, h]), ref[0]) < REL, (h, i)
