"""Bit-exact packed codes at the north-star scale: Llama-3-8B keys and values of
4 sequences x 8 kv heads x 32768 positions (1M rows, head_dim 128), bits 2/3/4,
plus GPT-2-shaped head_dim 64 at 98,304 rows and the query preparation of a
full 8192-token prefill.

The compression kernel is persistent: a block of 8 waves holds the weight
planes in LDS and walks 16-row tiles grid-stride, swapping Pi and Pi^T per
tile round for keys.  At 1M rows that is 32 rounds, so these cases cover every
round of every wave, the last partial tile included.  Bars (reference
compressors.py:114-138, :271-287): codes and sign bits equal the oracle's
packing of the device's own f32 rotated rows / projections byte for byte,
those f32 values agree with the oracle's f32 computation on every row, and the
f16 norms are within one f16 ulp.
"""

import math

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from test_gpu_kernels import _f16_ulps, _np
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

pytestmark = pytest.mark.gpu
DEV = "cuda"
CHUNK = 1 << 16  # rows per oracle pass


def _case(**kw):
    print("case:", kw, flush=True)


def _keys(shape, seed, outliers=True):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(*shape, device=DEV, generator=g)
    if outliers:
        x[..., :4] *= 20.0
    return x.to(torch.bfloat16)


def _check_keys(x, kc, ck, y_dev, p_dev):
    d = x.shape[-1]
    n = x.numel() // d
    pi, s = kc.Pi.cpu().numpy(), kc.S.cpu().numpy()
    cent, bounds = kc.centroids.cpu().numpy(), kc.boundaries.cpu().numpy()
    codes_dev = _np(ck["packed_key_indices"])
    signs_dev = _np(ck["packed_qjl_signs"])
    rn_dev = _np(ck["residual_norm"]).reshape(-1)
    vn_dev = _np(ck["vec_norms"]).reshape(-1)
    worst_dy, worst_proj, own_mismatch = 0.0, 0.0, 0
    for r0 in range(0, n, CHUNK):
        r1 = min(n, r0 + CHUNK)
        xs = x.reshape(n, d)[r0:r1].float().cpu().numpy()
        yd = _np(y_dev[r0:r1])
        pd = _np(p_dev[r0:r1])
        ref = O.key_compress_packed(xs, pi, s, cent, bounds, kc.mse_bits, y=yd)
        assert np.array_equal(codes_dev[r0:r1], ref["packed_key_indices"]), (r0, r1)
        assert np.array_equal(signs_dev[r0:r1], O.pack_bits((pd >= 0).astype(np.int32), 1)), (r0, r1)
        own = O.rotate(xs, pi)[2]
        worst_dy = max(worst_dy, float(np.max(np.abs(yd - own))))
        worst_proj = max(worst_proj, O.rel_err(pd, ref["proj"]))
        own_mismatch += int((O.quantize_searchsorted(own, bounds) != ref["codes"]).sum())
        assert _f16_ulps(vn_dev[r0:r1], ref["vec_norms"]).max() <= 1, (r0, r1)
        assert _f16_ulps(rn_dev[r0:r1], ref["residual_norm"]).max() <= 1, (r0, r1)
    print(f"rows {n}: max |dy| {worst_dy:.2e}, proj rel-err {worst_proj:.2e}, "
          f"codes from the oracle's own y differing {own_mismatch / (n * d):.2e}", flush=True)
    assert worst_dy < 2e-6 and worst_proj < 1e-5 and own_mismatch / (n * d) < 1e-3


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_key_codes_bit_exact_north_star(bits):
    shape = (4, 8, 32768, 128)
    _case(what="keys", shape=shape, bits=bits)
    x = _keys(shape, seed=100 + bits)
    kc = TurboQuantCompressorV2(128, bits, seed=42, device=DEV)
    n = x.numel() // 128
    y_dev = torch.empty(n, 128, device=DEV)
    p_dev = torch.empty(n, 128, device=DEV)
    ck = kc._compress_gpu(x, y_out=y_dev, proj_out=p_dev)
    torch.cuda.synchronize()
    _check_keys(x, kc, ck, y_dev, p_dev)


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_value_codes_bit_exact_north_star(bits):
    shape = (4, 8, 32768, 128)
    _case(what="values", shape=shape, bits=bits)
    x = _keys(shape, seed=200 + bits, outliers=False)
    vc = TurboQuantCompressorMSE(128, bits, seed=10042, device=DEV)
    n = x.numel() // 128
    y_dev = torch.empty(n, 128, device=DEV)
    cv = vc._compress_gpu(x, y_out=y_dev)
    torch.cuda.synchronize()
    pi, bounds = vc.Pi.cpu().numpy(), vc.boundaries.cpu().numpy()
    codes_dev = _np(cv["packed_indices"])
    vn_dev = _np(cv["vec_norms"])
    worst_dy, own_mismatch = 0.0, 0
    for r0 in range(0, n, CHUNK):
        r1 = min(n, r0 + CHUNK)
        xs = x.reshape(n, 128)[r0:r1].float().cpu().numpy()
        yd = _np(y_dev[r0:r1])
        ref = O.value_compress_packed(xs, pi, bounds, bits, y=yd)
        assert np.array_equal(codes_dev[r0:r1], ref["packed_indices"]), (r0, r1)
        assert _f16_ulps(vn_dev[r0:r1], ref["vec_norms"]).max() <= 1, (r0, r1)
        own = O.rotate(xs, pi)[2]
        worst_dy = max(worst_dy, float(np.max(np.abs(yd - own))))
        own_mismatch += int((O.quantize_searchsorted(own, bounds) != ref["codes"]).sum())
    print(f"rows {n}: max |dy| {worst_dy:.2e}, codes from own y differing {own_mismatch / (n * 128):.2e}",
          flush=True)
    assert worst_dy < 2e-6 and own_mismatch / (n * 128) < 1e-3


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_key_codes_bit_exact_head_dim_64(bits):
    shape = (8, 12, 1024, 64)  # 98,304 rows: GPT-2 small's head_dim, several tile rounds
    _case(what="keys d64", shape=shape, bits=bits)
    x = _keys(shape, seed=300 + bits)
    kc = TurboQuantCompressorV2(64, bits, seed=42, device=DEV)
    n = x.numel() // 64
    y_dev = torch.empty(n, 64, device=DEV)
    p_dev = torch.empty(n, 64, device=DEV)
    ck = kc._compress_gpu(x, y_out=y_dev, proj_out=p_dev)
    torch.cuda.synchronize()
    _check_keys(x, kc, ck, y_dev, p_dev)


def test_ragged_row_count_last_partial_tile():
    """A row count that is not a multiple of the 16-row tile, past one grid round."""
    shape = (1, 3, 12345, 128)
    _case(what="keys ragged", shape=shape)
    x = _keys(shape, seed=7)
    kc = TurboQuantCompressorV2(128, 3, seed=42, device=DEV)
    n = x.numel() // 128
    y_dev = torch.empty(n, 128, device=DEV)
    p_dev = torch.empty(n, 128, device=DEV)
    ck = kc._compress_gpu(x, y_out=y_dev, proj_out=p_dev)
    torch.cuda.synchronize()
    _check_keys(x, kc, ck, y_dev, p_dev)


def test_query_prep_at_prefill_scale():
    """q_rot (f16 rounding bound) and q_proj (f32 dot-product bound) of 32 heads x 8192 rows."""
    _case(what="query prep 262144 rows")
    g = torch.Generator(device=DEV).manual_seed(11)
    q = (torch.randn(1, 32, 8192, 128, device=DEV, generator=g) * 3).to(torch.bfloat16)
    kc = TurboQuantCompressorV2(128, 3, seed=42, device=DEV)
    q_rot, q_proj = kc.prepare_queries(q)
    torch.cuda.synchronize()
    pi = kc.Pi.cpu().numpy().astype(np.float64)
    se16 = _np(kc._dev_tables.s_eff16).astype(np.float64)
    qn = q.float().cpu().numpy().reshape(-1, 128).astype(np.float64)
    got = _np(q_rot).reshape(-1, 128).astype(np.float64)
    gp = _np(q_proj).reshape(-1, 128).astype(np.float64)
    for r0 in range(0, qn.shape[0], CHUNK):
        sl = slice(r0, r0 + CHUNK)
        exact = qn[sl] @ pi.T
        absum = np.abs(qn[sl]) @ np.abs(pi).T
        excess = (np.abs(got[sl] - exact) - (2.0 ** -11 * np.abs(exact) + 2.0 ** -25)) / absum
        assert excess.max() <= 2.0 ** -17, r0
        proj_ref = got[sl] @ se16.T
        proj_abs = np.abs(got[sl]) @ np.abs(se16).T
        assert np.all(np.abs(gp[sl] - proj_ref) <= 2.0 ** -24 * np.abs(proj_ref) + 2.0 ** -17 * proj_abs), r0
