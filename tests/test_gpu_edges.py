"""Edge shapes through the HIP path: empty sequences, no keys, no queries, one key.

The reference's PyTorch branch gives these shapes their torch meaning: compressing an
empty sequence yields empty planes, scores against no keys are an empty [.., S_q, 0]
tensor, and attention over no keys is softmax over an empty row followed by an empty
P.V product, i.e. zeros.  Each case here checks that meaning (and, where there is data,
the oracle) on the GPU kernels.
"""

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from turboquant_pytorch import compressed_attention
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2
from turboquant_pytorch.kernels import pack_bits, unpack_bits

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(**kw):
    print("case:", kw, flush=True)


@pytest.mark.parametrize("d", [64, 128])
def test_compress_empty_sequence(d):
    _case(what="compress S=0", d=d)
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, 3, seed=10042, device=DEV)
    x = torch.randn(2, 4, 0, d, device=DEV, dtype=torch.bfloat16)
    ck, cv = kc.compress(x), vc.compress(x)
    assert ck["packed_key_indices"].shape[0] == 0 and ck["packed_qjl_signs"].shape[0] == 0
    assert ck["residual_norm"].shape == (2, 4, 0) and ck["vec_norms"].shape == (2, 4, 0)
    assert cv["packed_indices"].shape[0] == 0 and cv["vec_norms"].numel() == 0
    assert vc.decompress(cv).numel() == 0


def test_pack_unpack_empty():
    _case(what="pack n=0")
    idx = torch.zeros(0, 128, dtype=torch.int32, device=DEV)
    packed = pack_bits(idx, 3)
    assert packed.shape == (0, O.pack_bits(np.zeros((0, 128), np.int32), 3).shape[1])
    assert unpack_bits(packed, 3, 128).shape == (0, 128)


@pytest.mark.parametrize("d,hq,hkv,sq", [(128, 32, 8, 1), (128, 8, 2, 37), (64, 4, 4, 5)])
def test_scores_and_attention_without_keys(d, hq, hkv, sq):
    _case(what="Sk=0", d=d, hq=hq, hkv=hkv, sq=sq)
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, 3, seed=10042, device=DEV)
    q = torch.randn(2, hq, sq, d, device=DEV, dtype=torch.bfloat16)
    kv = torch.randn(2, hkv, 0, d, device=DEV, dtype=torch.bfloat16)
    ck, cv = kc.compress(kv), vc.compress(kv)
    s = kc.asymmetric_attention_scores(q, ck)
    assert s.shape == (2, hq, sq, 0)
    o = compressed_attention(q, kc, vc, ck, cv, out_dtype=torch.float32)
    assert o.shape == (2, sq, hq, d)
    assert torch.count_nonzero(o).item() == 0


def test_attention_without_queries():
    _case(what="Sq=0")
    d = 128
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, 3, seed=10042, device=DEV)
    kv = torch.randn(1, 2, 50, d, device=DEV, dtype=torch.bfloat16)
    ck, cv = kc.compress(kv), vc.compress(kv)
    q = torch.randn(1, 8, 0, d, device=DEV, dtype=torch.bfloat16)
    assert kc.asymmetric_attention_scores(q, ck).shape == (1, 8, 0, 50)
    assert compressed_attention(q, kc, vc, ck, cv).shape == (1, 0, 8, d)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_single_key_is_its_value(causal):
    """With one key the softmax weight is exactly 1: the output is that key's decompressed value."""
    _case(what="Sk=1", causal=causal)
    d = 128
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, 3, seed=10042, device=DEV)
    torch.manual_seed(5)
    k = torch.randn(2, 2, 1, d, device=DEV, dtype=torch.bfloat16)
    v = torch.randn(2, 2, 1, d, device=DEV, dtype=torch.bfloat16)
    q = torch.randn(2, 8, 1, d, device=DEV, dtype=torch.bfloat16)
    ck, cv = kc.compress(k), vc.compress(v)
    o = compressed_attention(q, kc, vc, ck, cv, causal=causal, out_dtype=torch.float32).cpu().numpy()
    vals = vc.decompress(cv).float().cpu().numpy()  # [2, 2, 1, d]
    want = np.repeat(vals[:, :, 0, :], 4, axis=1)   # query head h reads kv head h // 4
    assert O.rel_err(o[:, 0], want) < 1e-3


def test_cache_empty_append_then_grow():
    """A zero-token append leaves an empty layer whose compact planes are empty; later appends
    match a one-shot compression."""
    _case(what="cache empty append")
    from transformers_turboquant import TurboQuantCache
    d, B, Hkv = 128, 1, 2
    kc = TurboQuantCompressorV2(d, 3, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, 3, seed=10042, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(3)
    k = torch.randn(B, Hkv, 20, d, device=DEV, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, 20, d, device=DEV, generator=g).to(torch.bfloat16)
    cache = TurboQuantCache()
    ck, cv = cache.append(0, kc, vc, k[:, :, :0], v[:, :, :0])
    assert ck["shape"] == (B, Hkv, 0, d)
    got_k, got_v = cache.layer(0).compact()
    assert got_k["packed_key_indices"].shape[0] == 0 and got_v["packed_indices"].shape[0] == 0
    cache.append(0, kc, vc, k, v)
    got_k, got_v = cache.layer(0).compact()
    fk, fv = kc.compress(k), vc.compress(v)
    assert torch.equal(got_k["packed_key_indices"], fk["packed_key_indices"])
    assert torch.equal(got_v["packed_indices"], fv["packed_indices"])
