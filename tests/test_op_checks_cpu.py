"""Argument checks of the torch.ops.tq layer, on the CPU.

Every op hands its planes and tables to the HIP library as raw pointers, so a
tensor on another device, of another dtype, non-contiguous (a sliced cache
plane) or shorter than the rows the kernels read must be refused before any
launch.  Each op's checks read tensor metadata only and are shared with its
Meta kernel (csrc/tq_torch.cpp), so these tests drive the same code with meta
tensors: no GPU and no kernel launch.  One well-formed call per op pins the
output shapes the Meta kernels report.
"""

import pytest
import torch

from turboquant_pytorch._ops import ops

M = "meta"
B, HQ, HKV, SQ, SK, D, BITS = 2, 8, 2, 3, 100, 128, 3
N = B * HKV * SK
F16, F32, U8 = torch.float16, torch.float32, torch.uint8


def _e(*shape, dtype=F32, device=M):
    return torch.empty(*shape, dtype=dtype, device=device)


def _keys(sk=SK, kv_stride=0, bits=BITS):
    rows = B * HKV * (kv_stride or sk)
    return dict(q_rot=_e(B, HQ, SQ, D, dtype=F16), q_proj=_e(B, HQ, SQ, D),
                codes=_e(rows, D * (bits - 1) // 8, dtype=U8), signs=_e(rows, D // 8, dtype=U8),
                rn=_e(rows, dtype=F16), vn=_e(rows, dtype=F16), cent=_e(1 << (bits - 1), dtype=F16))


def _scores(k, bits=BITS, hkv=HKV, sk=SK, kv_stride=0):
    return ops().scores(k["q_rot"], k["q_proj"], k["codes"], k["signs"], k["rn"], k["vn"], k["cent"], bits, hkv,
                        sk, kv_stride, 0.01)


def _values(sk=SK, kv_stride=0, bits=BITS):
    rows = B * HKV * (kv_stride or sk)
    return dict(vcodes=_e(rows, D * bits // 8, dtype=U8), vvn=_e(rows, dtype=F16), vcent=_e(1 << bits),
                vpit=_e(2, D, D, dtype=F16))


def _attention(k, v, mask=None, sk=SK, kv_stride=0, out_dtype=torch.bfloat16, workspace=1):
    return ops().attention(k["q_rot"], k["q_proj"], k["codes"], k["signs"], k["rn"], k["vn"], k["cent"], BITS,
                           v["vcodes"], v["vvn"], v["vcent"], BITS, v["vpit"], HKV, sk, kv_stride, 0.01, 0.088,
                           False, mask, out_dtype, workspace)


def _raises(match, fn, *a, **kw):
    with pytest.raises(RuntimeError, match=match):
        fn(*a, **kw)


def test_scores_shapes_and_kv_stride():
    assert _scores(_keys()).shape == (B, HQ, SQ, SK)
    # cache planes with capacity 256 per (batch, kv head): the last sequence needs only SK rows
    k = _keys(kv_stride=256)
    assert _scores(k, kv_stride=256).shape == (B, HQ, SQ, SK)
    rows = (B * HKV - 1) * 256 + SK
    for name in ("codes", "signs", "rn", "vn"):
        k2 = dict(k)
        k2[name] = k[name][:rows]
        _scores(k2, kv_stride=256)
        k2[name] = k[name][:rows - 1]
        _raises("the kernels read", _scores, k2, kv_stride=256)


@pytest.mark.parametrize("name,bad,match", [
    ("codes", lambda t: t[:-1], "the kernels read"),
    ("codes", lambda t: torch.empty(t.shape[0], 31, dtype=U8, device=M), "rows must hold 32"),
    ("codes", lambda t: t.to(torch.int8), "must be Byte"),
    ("signs", lambda t: t[:-1], "the kernels read"),
    ("signs", lambda t: torch.empty(t.shape[0], 32, dtype=U8, device=M)[:, ::2], "contiguous"),
    ("rn", lambda t: t.float(), "must be Half"),
    ("vn", lambda t: t[:-5], "the kernels read"),
    ("vn", lambda t: torch.empty(t.shape, dtype=F16), "is on cpu"),
    ("cent", lambda t: t[:2], "key centroids holds 2 elements"),
    ("cent", lambda t: t.float(), "must be Half"),
    ("q_proj", lambda t: t.half(), "q_proj float32"),
    ("q_proj", lambda t: torch.empty(B, HQ, SQ - 1, D, device=M), "differs from q_rot"),
    ("q_rot", lambda t: t.transpose(2, 3), "contiguous"),
])
def test_scores_refuses_bad_planes(name, bad, match):
    k = _keys()
    k[name] = bad(k[name])
    _raises(match, _scores, k)


def test_scores_refuses_bad_shapes():
    _raises("not a multiple", _scores, _keys(), hkv=3)
    _raises("kv_stride 50 must be 0 or at least", _scores, _keys(), kv_stride=50)
    _raises("key bits", _scores, _keys(), bits=1)


def test_attention_shapes_and_mask():
    k, v = _keys(), _values()
    assert _attention(k, v).shape == (B, SQ, HQ, D)
    assert _attention(k, v, out_dtype=torch.float32).dtype == torch.float32
    assert _attention(k, v, mask=_e(B, 1, SQ, SK)).shape == (B, SQ, HQ, D)
    assert _attention(k, v, mask=_e(SQ, SK)).shape == (B, SQ, HQ, D)
    _raises("expand", _attention, k, v, mask=_e(B, 1, SQ, SK + 1))
    _raises("broadcast", _attention, k, v, mask=_e(1, B, 1, SQ, SK))
    _raises("workspace mode", _attention, k, v, workspace=3)
    _raises("out_dtype", _attention, k, v, out_dtype=torch.int32)


@pytest.mark.parametrize("name,bad,match", [
    ("vcodes", lambda t: t[:-1], "the kernels read"),
    ("vcodes", lambda t: torch.empty(t.shape[0], 32, dtype=U8, device=M), "rows must hold 48"),
    ("vvn", lambda t: t[:-1], "the kernels read"),
    ("vvn", lambda t: t.float(), "must be Half"),
    ("vcent", lambda t: t[:4], "value centroids holds 4 elements"),
    ("vcent", lambda t: t.half(), "must be Float"),
    ("vpit", lambda t: t[:1], "split Pi_v"),
    ("vpit", lambda t: torch.empty(t.shape, dtype=F16), "is on cpu"),
])
def test_attention_refuses_bad_value_planes(name, bad, match):
    k, v = _keys(), _values()
    v[name] = bad(v[name])
    _raises(match, _attention, k, v)


def test_attention_refuses_bad_key_planes():
    k, v = _keys(), _values()
    k["rn"] = k["rn"][:-1]
    _raises("residual_norm", _attention, k, v)


def test_compress_ops():
    x = _e(B, HKV, SK, D, dtype=torch.bfloat16)
    pi, seff = _e(2, D, D, dtype=F16), _e(2, D, D, dtype=F16)
    cent, bnd = _e(4), _e(3)
    c, s, rn, vn = ops().compress_keys(x, pi, seff, cent, bnd, 2)
    assert c.shape == (N, 32) and s.shape == (N, 16) and rn.shape == (B, HKV, SK) and vn.dtype == F16
    ops().compress_keys(x, pi, seff, cent, bnd, 2, _e(N, D), _e(N, D))
    _raises("split Pi holds", ops().compress_keys, x, pi[:1], seff, cent, bnd, 2)
    _raises("split S_eff", ops().compress_keys, x, pi, seff.float(), cent, bnd, 2)
    _raises("centroids holds 2", ops().compress_keys, x, pi, seff, cent[:2], bnd, 2)
    _raises("boundaries", ops().compress_keys, x, pi, seff, cent, bnd[:2], 2)
    _raises("y_out", ops().compress_keys, x, pi, seff, cent, bnd, 2, _e(N - 1, D))
    _raises("proj_out", ops().compress_keys, x, pi, seff, cent, bnd, 2, None, _e(N, D, dtype=F16))

    c, vn = ops().compress_values(x, pi, _e(7), 3)
    assert c.shape == (N, 48) and vn.shape == (N,)
    _raises("boundaries", ops().compress_values, x, pi, _e(3), 3)
    _raises("y_out", ops().compress_values, x, pi, _e(7), 3, _e(N, D - 1))

    out = ops().decompress_values(c, vn, pi, _e(8), 3, [B, HKV, SK, D])
    assert out.shape == (B, HKV, SK, D) and out.dtype == F32
    _raises("packed_indices", ops().decompress_values, _e(N, 32, dtype=U8), vn, pi, _e(8), 3, [B, HKV, SK, D])
    _raises("value norms", ops().decompress_values, c, vn[:-1], pi, _e(8), 3, [B, HKV, SK, D])
    _raises("centroids holds 4", ops().decompress_values, c, vn, pi, _e(4), 3, [B, HKV, SK, D])

    qr, qp = ops().query_prep(_e(B, HQ, SQ, D), pi, _e(D, D, dtype=F16))
    assert qr.dtype == F16 and qp.dtype == F32 and qp.shape == (B, HQ, SQ, D)
    _raises("f16 S_eff", ops().query_prep, _e(B, HQ, SQ, D), pi, _e(D, D - 1, dtype=F16))


def test_kernel_function_ops():
    assert ops().pack_bits(_e(10, 7, dtype=torch.int32), 3).shape == (10, 3)
    _raises("b must be 1..8", ops().pack_bits, _e(10, 7, dtype=torch.int32), 9)
    assert ops().unpack_bits(_e(10, 3, dtype=U8), 3, 7).shape == (10, 7)
    _raises("hold fewer than", ops().unpack_bits, _e(10, 2, dtype=U8), 3, 7)
    assert ops().quantize_pack(_e(10, 128), _e(3), 2).shape == (10, 32)
    _raises("expected 3 boundaries", ops().quantize_pack, _e(10, 128), _e(4), 2)
    assert ops().dequantize(_e(10, 32, dtype=U8), _e(4), 2, 128).dtype == F16
    _raises("centroids for 2-bit", ops().dequantize, _e(10, 32, dtype=U8), _e(3), 2, 128)


def test_cache_ops():
    """tq::cache_append and tq::cache_attend (a cached decode step in one call) on meta tensors:
    output shapes, and the capacity, plane and query checks."""
    H, S, CAP, POS = HKV, 1, 64, 40
    k, v, q = _e(B, H, S, D), _e(B, H, S, D), _e(B, HQ, S, D)
    pi, seff, s16 = _e(2, D, D, dtype=F16), _e(2, D, D, dtype=F16), _e(D, D, dtype=F16)
    kcent, kbnd, vbnd = _e(1 << (BITS - 1)), _e((1 << (BITS - 1)) - 1), _e((1 << BITS) - 1)
    planes = [_e(B, H, CAP, D * (BITS - 1) // 8, dtype=U8), _e(B, H, CAP, D // 8, dtype=U8),
              _e(B, H, CAP, dtype=F16), _e(B, H, CAP, dtype=F16), _e(B, H, CAP, D * BITS // 8, dtype=U8),
              _e(B, H, CAP, dtype=F16)]
    head = (k, v, q, pi, seff, kcent, kbnd, BITS - 1, pi, vbnd, BITS, s16)
    qr, qp = ops().cache_append(*head, *planes, POS)
    assert qr.shape == (B, HQ, S, D) and qr.dtype == F16 and qp.dtype == F32
    tail = (_e(1 << (BITS - 1), dtype=F16), _e(1 << BITS), pi, 0.01, 0.1, True, None, torch.bfloat16, 1)
    out = ops().cache_attend(*head, *planes, POS, *tail)
    assert out.shape == (B, S, HQ, D) and out.dtype == torch.bfloat16
    _raises("exceed the capacity", ops().cache_attend, *head, *planes, CAP, *tail)
    _raises("q must be", ops().cache_attend, k, v, _e(B, HQ, S + 1, D), *head[3:], *planes, POS, *tail)
    bad = list(planes)
    bad[4] = _e(B, H, CAP, D * BITS // 8 - 1, dtype=U8)
    _raises("value codes", ops().cache_attend, *head, *bad, POS, *tail)
