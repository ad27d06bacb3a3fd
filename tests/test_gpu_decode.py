"""GPU parity of the split-K decode kernels (head_dim 64 / 128, at most 16 query
(row, head) columns per kv head) against the CPU oracle and the tiled kernel.

Same bars as the other kernel tests: scores and attention outputs within
rel-err 1e-3 and cosine >= 0.9999 of the float64 oracle estimator evaluated on
the device's packed planes.  Every case asserts first that the shape really
takes the decode path (non-zero workspace size).
"""

import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from test_gpu_kernels import _np, _oracle_attention, _oracle_scores, _planes
from turboquant_pytorch import _native, compressed_attention
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2
from turboquant_pytorch.kernels.attention import scores_from_prepared

pytestmark = pytest.mark.gpu
DEV = "cuda"
REL = 1e-3


def _case(**kw):
    print("case:", kw, flush=True)


def _on_decode_path(B, hq, hkv, sq, sk, bits, d=128):
    return _native.lib().tq_attention_workspace_size(B, hq, hkv, sq, sk, d, bits) > 0


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("hq,hkv,sq,sk", [
    (32, 8, 1, 4097), (8, 8, 1, 300), (16, 2, 2, 1000), (4, 1, 4, 65), (32, 8, 1, 1),
    (24, 4, 1, 2500), (16, 2, 1, 3000), (3, 1, 1, 999), (6, 2, 2, 513),
])
def test_decode_scores_match_oracle(bits, hq, hkv, sq, sk):
    _case(bits=bits, hq=hq, hkv=hkv, sq=sq, sk=sk)
    B, d = 2, 128
    assert _on_decode_path(B, hq, hkv, sq, sk, bits)
    torch.manual_seed(bits * 1000 + sk)
    k = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    q = torch.randn(B, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    ck = kc.compress(k)
    got = _np(kc.asymmetric_attention_scores(q, ck))
    ref = _oracle_scores(kc, q, ck, hq, hkv)
    assert got.shape == ref.shape
    assert O.rel_err(got, ref) < REL


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("cb", ["nonaffine", "shifted", "reference"])
@pytest.mark.parametrize("qmul", [1.0, 300.0, 1e-5])
@pytest.mark.parametrize("hq", [12, 8])
def test_decode_scores_any_codebook(bits, cb, qmul, hq):
    """Decode scores with key codebooks that are not odd (shifted, and for 2-bit codes
    not affine in the code bits: c3 - c2 != c1 - c0), and queries scaled far from 1,
    against the oracle evaluated with the same f16 codebook.  One query column is all
    zero.  6 and 4 columns per kv head (at bits 2-3 the bit-plane kernel's two- and
    one-group forms)."""
    _case(bits=bits, cb=cb, qmul=qmul, hq=hq)
    B, hkv, sq, sk, d = 2, 2, 1, 1500, 128
    assert _on_decode_path(B, hq, hkv, sq, sk, bits)
    torch.manual_seed(7 * bits + len(cb))
    k = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    q = torch.randn(B, hq, sq, d, device=DEV) * qmul
    q[1, 5] = 0.0
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    ck = kc.compress(k)
    cent = kc.centroids.cpu().double()
    if cb == "shifted":
        cent = cent + 0.3 * cent.abs().max()
    elif cb == "nonaffine":
        cent = cent * torch.linspace(0.6, 1.7, len(cent), dtype=torch.float64)
    cent16 = cent.to(torch.float16)
    q_rot, q_proj = kc.prepare_queries(q)
    got = _np(scores_from_prepared(q_rot, q_proj, ck["packed_key_indices"], ck["packed_qjl_signs"],
                                   ck["residual_norm"], ck["vec_norms"], cent16.to(DEV), bits,
                                   O.COEFF(d), hkv, sk))
    codes, signs, rn, vn = _planes(ck, d, kc.mse_bits)
    qr = _np(q_rot.float()).reshape(B, hq, sq, d)
    qp = _np(q_proj).reshape(B, hq, sq, d)
    ref = np.zeros((B, hq, sq, sk))
    for b in range(B):
        for h in range(hq):
            r = slice((b * hkv + h // (hq // hkv)) * sk, (b * hkv + h // (hq // hkv) + 1) * sk)
            ref[b, h] = O.scores_packed(qr[b, h], qp[b, h], codes[r], signs[r], rn[r], vn[r],
                                        cent16.numpy(), O.COEFF(d))
    assert np.all(got[1, 5] == 0.0)
    assert O.rel_err(got, ref) < REL, O.rel_err(got, ref)


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("cb", ["nonaffine", "shifted"])
@pytest.mark.parametrize("hq", [8, 16])
@pytest.mark.parametrize("d", [128, 64])
def test_decode_attention_any_codebook(bits, cb, hq, d):
    """Fused decode attention with key codebooks that are not odd (and, for 2-bit codes, not
    affine in the code bits) against the oracle evaluated with the same f16 codebook; 4 and 8
    columns per kv head (one and two column groups of the bit-plane kernel), head_dim 128
    and 64."""
    _case(bits=bits, cb=cb, hq=hq, d=d)
    from turboquant_pytorch._ops import ops
    from turboquant_pytorch.compressors import _tables

    B, hkv, sq, sk = 2, 2, 1, 2000
    assert _on_decode_path(B, hq, hkv, sq, sk, bits, d)
    torch.manual_seed(11 * bits + len(cb))
    q = torch.randn(B, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    cent = kc.centroids.cpu().double()
    cent = cent + 0.3 * cent.abs().max() if cb == "shifted" else cent * torch.linspace(0.6, 1.7, len(cent), dtype=torch.float64)
    cent16 = cent.to(torch.float16)
    q_rot, q_proj = kc.prepare_queries(q)
    tv = _tables(vc, q.device, with_qjl=False)
    got = _np(ops().attention(q_rot, q_proj, ck["packed_key_indices"], ck["packed_qjl_signs"], ck["residual_norm"],
                              ck["vec_norms"], cent16.to(DEV), bits, cv["packed_indices"], cv["vec_norms"], tv.cent32,
                              vc.bits, tv.pit_split, hkv, sk, sk, O.COEFF(d), 1 / math.sqrt(d), False, None,
                              torch.float32, 1))
    codes, signs, rn, vn = _planes(ck, d, kc.mse_bits)
    qr = _np(q_rot.float()).reshape(B, hq, sq, d)
    qp = _np(q_proj).reshape(B, hq, sq, d)
    codes_v = O.unpack_bits(_np(cv["packed_indices"]), vc.bits, d)
    vals = O.value_decompress(codes_v, _np(cv["vec_norms"]).reshape(-1), vc.Pi.cpu().numpy(),
                              vc.centroids.cpu().numpy()).reshape(B, hkv, sk, d)
    ref = np.zeros((B, sq, hq, d))
    g = hq // hkv
    for b in range(B):
        for h in range(hq):
            r = slice((b * hkv + h // g) * sk, (b * hkv + h // g + 1) * sk)
            sc = O.scores_packed(qr[b, h], qp[b, h], codes[r], signs[r], rn[r], vn[r], cent16.numpy(), O.COEFF(d))
            ref[b, :, h] = O.attention(sc, vals[b, h // g], 1 / math.sqrt(d))
    assert O.rel_err(got, ref) < REL, O.rel_err(got, ref)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("hq,hkv,sq,sk,causal,qmul,vmul", [
    (32, 8, 1, 5000, False, 1.0, 1.0),
    (8, 2, 4, 1025, True, 1.0, 1.0),     # last split holds one key: fully masked for rows 0-2
    (4, 4, 1, 1, False, 1.0, 1.0),
    (16, 1, 1, 700, True, 8.0, 1.0),     # sharp softmax, 16 heads per kv head
    (2, 1, 8, 3000, True, 1.0, 3000.0),  # value norms ~3e4: near the f16 range
    (8, 4, 2, 1025, True, 1.0, 1.0),     # 4 columns (2 heads x 2 rows), causal
    (12, 4, 1, 3001, False, 8.0, 3000.0),
    (6, 2, 1, 2048, True, 1.0, 0.01),
    (16, 2, 1, 5000, False, 1.0, 1.0),   # 8 columns: two column groups of the bit-plane kernel
    (8, 2, 2, 1025, True, 1.0, 1.0),     # 8 columns (4 heads x 2 rows), causal
    (5, 1, 1, 777, False, 8.0, 1.0),     # 5 columns: the second group holds one
    (12, 2, 1, 3001, True, 1.0, 3000.0), # 6 columns, value norms ~3e4
    (16, 2, 1, 20000, True, 1.0, 1.0),   # 8 columns, 79 splits: the merge with one block per column
])
def test_decode_attention_matches_oracle_and_tiled(bits, hq, hkv, sq, sk, causal, qmul, vmul):
    _case(bits=bits, hq=hq, hkv=hkv, sq=sq, sk=sk, causal=causal, qmul=qmul, vmul=vmul)
    B, d = 2, 128
    assert _on_decode_path(B, hq, hkv, sq, sk, bits)
    torch.manual_seed(bits + 3 * sk)
    q = torch.randn(B, hq, sq, d, device=DEV, dtype=torch.bfloat16) * qmul
    k = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16) * vmul
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    got = _np(compressed_attention(q, kc, vc, ck, cv, causal=causal, out_dtype=torch.float32))
    tiled = _np(compressed_attention(q, kc, vc, ck, cv, causal=causal, out_dtype=torch.float32, split_k=False))
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, causal=causal)
    assert np.isfinite(got).all()
    print(f"ERR decode {O.rel_err(got, ref):.2e} cos {1 - O.cosine(got, ref):.1e} tiled {O.rel_err(tiled, ref):.2e}")
    assert O.rel_err(got, ref) < REL and O.cosine(got, ref) > 0.9999
    assert O.rel_err(tiled, ref) < REL


@pytest.mark.parametrize("hq,hkv,sq", [(8, 2, 2), (4, 2, 2)])
def test_decode_attention_mask_and_dtypes(hq, hkv, sq):
    _case(what="decode mask", hq=hq, hkv=hkv, sq=sq)
    torch.manual_seed(12)
    B, sk, d = 2, 600, 128
    assert _on_decode_path(B, hq, hkv, sq, sk, 3)
    q = torch.randn(B, hq, sq, d, device=DEV)
    k = torch.randn(B, hkv, sk, d, device=DEV)
    v = torch.randn(B, hkv, sk, d, device=DEV)
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, 3, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    mask = torch.zeros(B, 1, sq, sk)
    mask[0, 0, :, 400:] = torch.finfo(torch.float32).min  # padding on batch 0
    mask[1, 0, 1, :37] = -5.0
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, mask=mask.numpy())
    for dt in (torch.float32, torch.bfloat16, torch.float16):
        got = compressed_attention(q.to(dt), kc, vc, ck, cv, attention_mask=mask.to(DEV), out_dtype=dt)
        tol = REL if dt == torch.float32 else 8e-3
        assert O.rel_err(_np(got.float()), ref) < tol


def test_decode_long_context_slice():
    """Decode at the headline shape (4 sequences x 32k keys, 8 kv / 32 q heads, bits=3);
    oracle on a few (sequence, head) pairs."""
    _case(what="decode 32k")
    torch.manual_seed(1)
    B, hq, hkv, sk, d = 4, 32, 8, 32768, 128
    assert _on_decode_path(B, hq, hkv, 1, sk, 3)
    q = torch.randn(B, hq, 1, d, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    k[..., :4] *= 20
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, 3, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    out = compressed_attention(q, kc, vc, ck, cv, causal=True, out_dtype=torch.float32)
    tiled = compressed_attention(q, kc, vc, ck, cv, causal=True, out_dtype=torch.float32, split_k=False)
    assert torch.isfinite(out).all()
    codes, signs, rn, vn = _planes(ck, d, kc.mse_bits)
    codes_v = O.unpack_bits(_np(cv["packed_indices"]), 3, d)
    q_rot, q_proj = O.query_prep(q.float().cpu().numpy(), kc.Pi.cpu().numpy(), kc._dev_tables.s_eff16.cpu().numpy())
    q_rot = q_rot.reshape(B, hq, d)
    q_proj = q_proj.reshape(B, hq, d)
    cent16 = kc.centroids.cpu().numpy().astype(np.float16)
    for b, h in ((0, 0), (1, 13), (3, 31)):
        kv = b * hkv + h // 4
        r = slice(kv * sk, (kv + 1) * sk)
        sc = O.scores_packed(q_rot[b, h][None], q_proj[b, h][None], codes[r], signs[r], rn[r], vn[r],
                             cent16, O.COEFF(d))
        vals = O.value_decompress(codes_v[r], _np(cv["vec_norms"]).reshape(-1)[r], vc.Pi.cpu().numpy(),
                                  vc.centroids.cpu().numpy())
        ref = O.attention(sc, vals, 1 / math.sqrt(d))[0]
        assert O.rel_err(_np(out[b, 0, h]), ref) < REL, (b, h)
        assert O.rel_err(_np(tiled[b, 0, h]), ref) < REL, (b, h)


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("sk,vmul", [(16384, 1.0), (32768, 1.0), (32768, 0.01)])
def test_decode_attention_sink_keeps_small_weights(bits, sk, vmul):
    """One sink key ~12 nats above 16-32k ordinary keys: the ordinary keys' weights are
    e^-12 of the sink's each, yet together they carry a fifth to a third of the mass.
    Each must reach P.V, not only the f32 normaliser (small value norms included)."""
    _case(what="sink", bits=bits, sk=sk, vmul=vmul)
    B, hq, hkv, d = 1, 4, 1, 128
    assert _on_decode_path(B, hq, hkv, 1, sk, bits)
    g = torch.Generator().manual_seed(sk + bits)
    u = torch.randn(d, generator=g)
    q = (u + 0.05 * torch.randn(B, hq, 1, d, generator=g)).to(DEV)
    k = torch.randn(B, hkv, sk, d, generator=g)
    sink = 777
    k[0, 0, sink] = 12.0 * math.sqrt(d) * u / (u @ u)  # score q.k / sqrt(d) ~ 12
    v = (torch.randn(B, hkv, sk, d, generator=g) * vmul)
    k, v = k.to(DEV), v.to(DEV)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    got = _np(compressed_attention(q, kc, vc, ck, cv, out_dtype=torch.float32))
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv)
    sc = _oracle_scores(kc, q, ck, hq, hkv)[0, 0, 0] / math.sqrt(d)
    w = np.exp(sc - sc.max())
    share = 1 - w[sink] / w.sum()
    print(f"ordinary keys' share of the weight {share:.3f}; rel-err {O.rel_err(got, ref):.2e}", flush=True)
    assert sc.argmax() == sink and 0.1 < share < 0.6
    assert O.rel_err(got, ref) < REL and O.cosine(got, ref) > 0.9999


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("sq,npad", [(1, 64), (1, 200), (1, 1000), (2, 100)])
def test_decode_attention_left_padding(bits, sq, npad):
    """Left padding with finfo.min on the first `npad` keys of batch row 0: whole 32-key slabs,
    and at npad = 1000 whole splits, see only masked keys before the first real one.  Batch row
    1 masks one key with a moderate bias, batch row 2 masks every key (the reference's softmax
    of equal scores gives every key the same weight).  At bits 2-3, Sq = 1 takes the bit-plane
    kernel's one-group form (4 columns) and Sq = 2 its two-group form (8 columns); bits 4 the
    table kernel.  Against the float64 oracle."""
    _case(what="decode left padding", bits=bits, sq=sq, npad=npad)
    B, hq, hkv, sk, d = 3, 16, 4, 1500, 128
    assert _on_decode_path(B, hq, hkv, sq, sk, bits)
    torch.manual_seed(31 * bits + npad + sq)
    q = torch.randn(B, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    fmin = torch.finfo(torch.float32).min
    mask = torch.zeros(B, 1, sq, sk)
    mask[0, 0, :, :npad] = fmin
    mask[1, 0, :, 5] = -3.0
    mask[2] = fmin
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, mask=mask.numpy())
    got = _np(compressed_attention(q, kc, vc, ck, cv, attention_mask=mask.to(DEV), out_dtype=torch.float32))
    assert np.isfinite(got).all()
    for b in range(B):
        err = O.rel_err(got[b], ref[b])
        print(f"batch row {b}: rel-err {err:.2e}", flush=True)
        assert err < REL, (b, err)


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("hq,hkv,sq,sk,causal,masked", [
    (5, 1, 1, 2000, False, False),   # 5 columns: one lane group of the second column group
    (7, 1, 1, 9000, False, True),    # 7 columns, padding mask, 36 splits (merge by column blocks)
    (3, 1, 2, 1500, True, False),    # 6 columns from 3 heads x 2 rows, causal
    (14, 2, 1, 20000, True, False),  # 7 columns per kv head over 2 kv heads, many splits
])
def test_decode_two_column_groups_scores_and_attention(bits, hq, hkv, sq, sk, causal, masked):
    """Bit-plane decode kernels with 5-8 columns per kv head (the second column group partly
    filled), scores and fused attention against the float64 oracle, with the merge of few and
    of many splits."""
    _case(bits=bits, hq=hq, hkv=hkv, sq=sq, sk=sk, causal=causal, masked=masked)
    B, d = 2, 128
    assert _on_decode_path(B, hq, hkv, sq, sk, bits)
    torch.manual_seed(17 * bits + hq + sk)
    q = torch.randn(B, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    got_s = _np(kc.asymmetric_attention_scores(q, ck))
    ref_s = _oracle_scores(kc, q, ck, hq, hkv)
    assert O.rel_err(got_s, ref_s) < REL
    mask = None
    if masked:
        mask = torch.zeros(B, 1, sq, sk)
        mask[0, 0, :, : sk // 3] = torch.finfo(torch.float32).min  # left padding on batch row 0
        mask[1, 0, :, 7] = -4.0
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, causal=causal,
                            mask=mask.numpy() if mask is not None else None)
    got = _np(compressed_attention(q, kc, vc, ck, cv, causal=causal, out_dtype=torch.float32,
                                   attention_mask=mask.to(DEV) if mask is not None else None))
    assert np.isfinite(got).all()
    err = O.rel_err(got, ref)
    print(f"scores rel-err {O.rel_err(got_s, ref_s):.2e}, attention rel-err {err:.2e}", flush=True)
    assert err < REL and O.cosine(got, ref) > 0.9999


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("hq,hkv,sq,sk,causal,masked", [
    (32, 8, 1, 4097, False, False),   # 4 columns per kv head (a 32/8-head model)
    (12, 12, 1, 3000, False, False),  # one column per kv head (multi-head attention)
    (16, 2, 1, 20000, True, False),   # 8 columns, 79 splits
    (8, 2, 2, 1025, True, True),      # 8 columns from 4 heads x 2 rows, causal, mask
    (5, 1, 1, 777, False, False),     # 5 columns: the second group holds one
    (4, 1, 1, 1, False, False),       # a single key
    (6, 2, 1, 65, True, False),       # 3 columns, one partial slab
    (7, 1, 1, 9000, False, True),     # 7 columns, padding mask
    (16, 1, 1, 3000, False, False),   # 16 columns: the table kernels at every width
    (6, 2, 4, 1500, True, False),     # 12 columns from 3 heads x 4 rows, causal
    (24, 2, 1, 20000, True, True),    # 12 columns, 79 splits, padding mask
])
def test_decode_head_dim64_scores_and_attention(bits, hq, hkv, sq, sk, causal, masked):
    """The decode kernels at head_dim 64: the bit-plane kernels (bits 2-3, at most 8 columns;
    16-dim lane groups: 2-byte sign and 1-bit code fields, 4 value dims per lane) and the
    table kernels (bits 4, or 9-16 columns; 6-byte code fields at bits 4), scores and fused
    attention against the float64 oracle, and the tiled kernel on the same inputs."""
    _case(what="decode d64", bits=bits, hq=hq, hkv=hkv, sq=sq, sk=sk, causal=causal, masked=masked)
    B, d = 2, 64
    assert _on_decode_path(B, hq, hkv, sq, sk, bits, d)
    torch.manual_seed(29 * bits + hq + sk)
    q = torch.randn(B, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    k = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(B, hkv, sk, d, device=DEV, dtype=torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    got_s = _np(kc.asymmetric_attention_scores(q, ck))
    ref_s = _oracle_scores(kc, q, ck, hq, hkv)
    assert got_s.shape == ref_s.shape
    assert O.rel_err(got_s, ref_s) < REL
    mask = None
    if masked:
        mask = torch.zeros(B, 1, sq, sk)
        mask[0, 0, :, : sk // 3] = torch.finfo(torch.float32).min  # left padding on batch row 0
        mask[1, 0, :, 7] = -4.0
    mask_dev = mask.to(DEV) if mask is not None else None
    ref = _oracle_attention(kc, vc, q, ck, cv, hq, hkv, causal=causal,
                            mask=mask.numpy() if mask is not None else None)
    got = _np(compressed_attention(q, kc, vc, ck, cv, causal=causal, out_dtype=torch.float32,
                                   attention_mask=mask_dev))
    tiled = _np(compressed_attention(q, kc, vc, ck, cv, causal=causal, out_dtype=torch.float32,
                                     attention_mask=mask_dev, split_k=False))
    assert np.isfinite(got).all()
    err = O.rel_err(got, ref)
    print(f"scores rel-err {O.rel_err(got_s, ref_s):.2e}, attention rel-err {err:.2e}, "
          f"tiled {O.rel_err(tiled, ref):.2e}", flush=True)
    assert err < REL and O.cosine(got, ref) > 0.9999
    assert O.rel_err(tiled, ref) < REL
