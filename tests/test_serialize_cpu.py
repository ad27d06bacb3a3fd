"""Serialization of compressed KV planes (format turboquant-kv v1).

The committed fixture tests/golden/kv_format_v1.safetensors pins the on-disk
format: it must load into exactly the planes its generator describes.  Round
trips must be bit-exact for both layouts, and malformed or newer containers
must be refused with FormatError.
"""

import json
import os
import sys

import pytest
import torch

from transformers_turboquant import TurboQuantCache, apply_turboquant
from turboquant_pytorch import serialize as SZ
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
sys.path.insert(0, GOLDEN)
import make_kv_format  # noqa: E402


def _equal(a: dict, b: dict):
    assert set(a) == set(b), (set(a), set(b))
    for k in a:
        if k == "shape":
            assert tuple(a[k]) == tuple(b[k])
        else:
            assert a[k].dtype == b[k].dtype and torch.equal(a[k].reshape(b[k].shape), b[k]), k


def test_golden_fixture_loads():
    groups, user = SZ.load_groups(os.path.join(GOLDEN, "kv_format_v1.safetensors"))
    assert user == {"note": "format fixture"}
    want = make_kv_format.planes()
    assert [g["name"] for g in groups] == ["p", "u"]
    p, u = groups
    _equal(p["keys"], want[0]["keys"])
    _equal(p["values"], want[0]["values"])
    assert (p["key_bits"], p["value_bits"], p["key_seed"], p["value_seed"]) == (3, 3, 7, 10007)
    assert p["keys"]["residual_norm"].shape == (1, 2, 3) and p["values"]["vec_norms"].shape == (6,)
    _equal(u["keys"], want[1]["keys"])
    assert u["values"] is None and u["value_bits"] is None


def _random_packed(B, H, S, D, bits, seed=0):
    g = torch.Generator().manual_seed(seed)
    n = B * H * S
    kc = -(-D * max(bits - 1, 1) // 8)
    k = {"packed_key_indices": torch.randint(0, 256, (n, kc), generator=g, dtype=torch.uint8),
         "packed_qjl_signs": torch.randint(0, 256, (n, D // 8), generator=g, dtype=torch.uint8),
         "residual_norm": torch.rand(B, H, S, generator=g).half(),
         "vec_norms": torch.rand(B, H, S, generator=g).half(), "shape": (B, H, S, D)}
    v = {"packed_indices": torch.randint(0, 256, (n, -(-D * bits // 8)), generator=g, dtype=torch.uint8),
         "vec_norms": torch.rand(n, generator=g).half(), "shape": (B, H, S, D)}
    return k, v


@pytest.mark.parametrize("D,bits", [(64, 2), (128, 3), (128, 4), (256, 3)])
def test_packed_roundtrip_bytes_and_file(tmp_path, D, bits):
    k, v = _random_packed(2, 3, 17, D, bits, seed=D + bits)
    kc = TurboQuantCompressorV2(D, bits, seed=5)
    vc = TurboQuantCompressorMSE(D, bits, seed=10005)
    data = SZ.dumps(k, v, kc, vc, metadata={"model": "x"})
    k2, v2, info = SZ.loads(data)
    _equal(k2, k)
    _equal(v2, v)
    assert info == {"key_bits": bits, "value_bits": bits, "key_seed": 5, "value_seed": 10005, "model": "x"}
    path = tmp_path / "kv.safetensors"
    SZ.save_compressed(path, k, v, kc, vc)
    k3, v3, _ = SZ.load_compressed(path)
    _equal(k3, k)
    _equal(v3, v)
    assert os.path.getsize(path) == len(SZ.dumps(k, v, kc, vc))


def test_bits_inferred_without_compressors():
    k, v = _random_packed(1, 2, 5, 128, 4)
    _, _, info = SZ.loads(SZ.dumps(k, v))
    assert info["key_bits"] == 4 and info["value_bits"] == 4 and info["key_seed"] is None


def test_unpacked_roundtrip_scores_unchanged():
    kc = TurboQuantCompressorV2(64, 3, seed=1)
    vc = TurboQuantCompressorMSE(64, 3, seed=10001)
    g = torch.Generator().manual_seed(2)
    x = torch.randn(2, 2, 9, 64, generator=g)
    ck, cv = kc.compress(x), vc.compress(x)
    k2, v2, _ = SZ.loads(SZ.dumps(ck, cv, kc, vc))
    _equal(k2, ck)
    _equal(v2, cv)
    q = torch.randn(2, 2, 3, 64, generator=g)
    assert torch.equal(kc.asymmetric_attention_scores(q, k2), kc.asymmetric_attention_scores(q, ck))
    assert torch.equal(vc.decompress(v2), vc.decompress(cv))


def test_keys_only_and_values_only():
    k, v = _random_packed(1, 1, 4, 32, 3)
    k2, v2, _ = SZ.loads(SZ.dumps(keys=k))
    _equal(k2, k)
    assert v2 is None
    k3, v3, _ = SZ.loads(SZ.dumps(values=v))
    assert k3 is None
    _equal(v3, v)


def _rewrite(data: bytes, edit) -> bytes:
    n = int.from_bytes(data[:8], "little")
    head = json.loads(data[8:8 + n])
    edit(head)
    raw = json.dumps(head).encode()
    raw += b" " * (-len(raw) % 8)
    return len(raw).to_bytes(8, "little") + raw + data[8 + n:]


def test_rejects_malformed():
    k, v = _random_packed(1, 2, 3, 32, 3)
    good = SZ.dumps(k, v)
    SZ.loads(_rewrite(good, lambda h: None))  # the rewriter itself keeps a valid container

    def meta(key, val):
        return lambda h: h["__metadata__"].__setitem__(key, val)

    def group(key, val):
        def f(h):
            gs = json.loads(h["__metadata__"]["groups"])
            gs[0][key] = val
            h["__metadata__"]["groups"] = json.dumps(gs)
        return f

    cases = [meta("format", "other"), meta("version", "2"), meta("version", "x"), meta("groups", "{"),
             group("shape", [1, 2, 4, 32]), group("key_bits", 4), group("layout", "dense"),
             lambda h: h.pop("kv/v.vn"), lambda h: h["__metadata__"].pop("groups")]
    for edit in cases:
        with pytest.raises(SZ.FormatError):
            SZ.loads(_rewrite(good, edit))
    with pytest.raises(SZ.FormatError):
        SZ.loads(good[:5])
    with pytest.raises(SZ.FormatError):
        SZ.loads(good[:-7])
    with pytest.raises(SZ.FormatError):
        SZ.loads(b"\x10\x00\x00\x00\x00\x00\x00\x00not json at all!")


def test_writer_rejects_inconsistent_planes():
    k, v = _random_packed(1, 2, 3, 32, 3)
    bad = dict(k, packed_qjl_signs=k["packed_qjl_signs"][:, :3])
    with pytest.raises(ValueError):
        SZ.dumps(bad, v)
    with pytest.raises(ValueError):
        SZ.dumps(k, dict(v, shape=(1, 2, 4, 32)))
    with pytest.raises(ValueError):
        SZ.dumps(k, {"indices": torch.zeros(6, 32, dtype=torch.uint8), "vec_norms": torch.zeros(6).half(),
                     "shape": (1, 2, 3, 32)})


def test_cache_save_load_continues_generation(tmp_path):
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(0)
    cfg = LlamaConfig(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2)
    model = apply_turboquant(LlamaForCausalLM(cfg).eval(), bits=3, seed=42)
    ids = torch.randint(0, 128, (2, 11), generator=torch.Generator().manual_seed(3))
    kw = dict(do_sample=False)
    with torch.no_grad():
        full = model.generate(ids, max_new_tokens=6, min_new_tokens=6, past_key_values=TurboQuantCache(), **kw)
        cache = TurboQuantCache()
        part = model.generate(ids, max_new_tokens=3, min_new_tokens=3, past_key_values=cache, **kw)
        path = tmp_path / "cache.safetensors"
        cache.save(path, metadata={"model": "tiny-llama"})
        loaded = TurboQuantCache.load(path)
        assert loaded.get_seq_length() == cache.get_seq_length() == 13
        for a, b in zip(cache.layers, loaded.layers):
            _equal(b.cpu_k, a.cpu_k)
            _equal(b.cpu_v, a.cpu_v)
            assert b.codec == a.codec and a.codec["key_seed"] is not None
        rest = model.generate(part, max_new_tokens=3, min_new_tokens=3, past_key_values=loaded, **kw)
    assert torch.equal(rest, full)


def test_cache_load_rejects_packed_on_cpu(tmp_path):
    k, v = _random_packed(1, 2, 3, 32, 3)
    path = tmp_path / "c.safetensors"
    SZ.save_groups(path, [{"name": "layer0", "keys": k, "values": v}])
    with pytest.raises(ValueError):
        TurboQuantCache.load(path, device="cpu")
    SZ.save_groups(path, [{"name": "kv", "keys": k, "values": v}])
    with pytest.raises(SZ.FormatError):
        TurboQuantCache.load(path, device="cpu")


def test_writer_reproduces_fixture_bytes(tmp_path):
    """The writer is deterministic across processes (the container's metadata keys are emitted
    sorted), so the fixture's planes written now give the committed file byte for byte."""
    out = tmp_path / "again.safetensors"
    SZ.save_groups(out, make_kv_format.planes(), metadata={"note": "format fixture"})
    with open(os.path.join(GOLDEN, "kv_format_v1.safetensors"), "rb") as f:
        assert out.read_bytes() == f.read()
