"""Serialized packed planes on the GPU: a save/load round trip changes nothing.

Planes written from the GPU compressors and loaded back onto the device must be
the same bytes, attention over them must give the same result bit for bit, and
a cache restored from a file must continue greedy decoding exactly as the
uninterrupted cache does.
"""

import pytest
import torch

from transformers_turboquant import TurboQuantCache, apply_turboquant
from turboquant_pytorch import serialize as SZ
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2
from turboquant_pytorch.fused import compressed_attention

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_gpu_planes_roundtrip(bits):
    print("case: serialize planes bits", bits, flush=True)
    dev, d = "cuda", 128
    kc = TurboQuantCompressorV2(d, bits, seed=3, device=dev)
    vc = TurboQuantCompressorMSE(d, bits, seed=10003, device=dev)
    g = torch.Generator(device=dev).manual_seed(bits)
    k = torch.randn(2, 2, 300, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(2, 2, 300, d, device=dev, generator=g).to(torch.bfloat16)
    ck, cv = kc.compress(k), vc.compress(v)
    k2, v2, info = SZ.loads(SZ.dumps(ck, cv, kc, vc), device=dev)
    assert info["key_seed"] == 3 and info["value_bits"] == bits
    for name in ("packed_key_indices", "packed_qjl_signs", "residual_norm", "vec_norms"):
        assert k2[name].device.type == "cuda" and torch.equal(k2[name], ck[name]), name
    for name in ("packed_indices", "vec_norms"):
        assert torch.equal(v2[name], cv[name]), name
    for sq in (1, 37):
        q = torch.randn(2, 8, sq, d, device=dev, generator=g).to(torch.bfloat16)
        a = compressed_attention(q, kc, vc, ck, cv, causal=True, out_dtype=torch.float32)
        b = compressed_attention(q, kc, vc, k2, v2, causal=True, out_dtype=torch.float32)
        torch.cuda.synchronize()
        assert torch.equal(a, b), sq


def test_gpu_cache_save_load_continues_generation(tmp_path):
    print("case: serialize cache gpu", flush=True)
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(0)
    cfg = LlamaConfig(vocab_size=1000, hidden_size=1024, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2)
    model = apply_turboquant(LlamaForCausalLM(cfg).eval(), bits=3).to("cuda", torch.float32)
    ids = torch.randint(0, 1000, (2, 300), generator=torch.Generator().manual_seed(5)).cuda()
    kw = dict(do_sample=False, attention_mask=None)
    with torch.no_grad():
        full = model.generate(ids, max_new_tokens=6, min_new_tokens=6, past_key_values=TurboQuantCache(), **kw)
        cache = TurboQuantCache()
        part = model.generate(ids, max_new_tokens=3, min_new_tokens=3, past_key_values=cache, **kw)
        path = tmp_path / "cache.safetensors"
        cache.save(path)
        loaded = TurboQuantCache.load(path, device="cuda")
        assert loaded.get_seq_length() == 302
        for a, b in zip(cache.layers, loaded.layers):
            ka, va = a.compact()
            kb, vb = b.compact()
            for name in ka:
                if name != "shape":
                    assert torch.equal(ka[name], kb[name]), name
            for name in va:
                if name != "shape":
                    assert torch.equal(va[name], vb[name]), name
        rest = model.generate(part, max_new_tokens=3, min_new_tokens=3, past_key_values=loaded, **kw)
    assert torch.equal(rest, full)


def _to(groups, device):
    out = []
    for g in groups:
        g = dict(g)
        for which in ("keys", "values"):
            if g.get(which) is not None:
                g[which] = {k: (v if k == "shape" else v.to(device)) for k, v in g[which].items()}
        out.append(g)
    return out


def test_gpu_golden_format_fixture(tmp_path):
    """The committed format fixture (tests/golden/kv_format_v1.safetensors) read straight onto
    the GPU holds exactly the planes its generator describes, and the same planes written from
    device tensors give a file byte-identical to the committed one."""
    print("case: serialize golden fixture on gpu", flush=True)
    import os
    import sys

    golden = os.path.join(os.path.dirname(__file__), "golden")
    sys.path.insert(0, golden)
    import make_kv_format

    path = os.path.join(golden, "kv_format_v1.safetensors")
    groups, user = SZ.load_groups(path, device="cuda")
    assert user == {"note": "format fixture"}
    want = _to(make_kv_format.planes(), "cuda")
    assert [g["name"] for g in groups] == [g["name"] for g in want]
    for got, exp in zip(groups, want):
        for which in ("keys", "values"):
            if exp.get(which) is None:
                assert got[which] is None
                continue
            assert set(got[which]) == set(exp[which]), which
            for name, t in exp[which].items():
                if name == "shape":
                    assert tuple(got[which][name]) == tuple(t)
                    continue
                g = got[which][name]
                assert g.device.type == "cuda" and g.dtype == t.dtype, (which, name)
                assert torch.equal(g.reshape(t.shape), t), (which, name)
    out = tmp_path / "from_gpu.safetensors"
    SZ.save_groups(out, want, metadata={"note": "format fixture"})
    with open(path, "rb") as f:
        committed = f.read()
    assert out.read_bytes() == committed
