"""Host-side API on CPU tensors: compressors, kernel functions, registry, patching.

CPU tensors follow the reference's PyTorch branch, whose outputs are pinned by
the reference's own golden vectors (tests/golden/cpu_compress.npz,
gpt2_logits.npz) and by the oracle.
"""

import math
import os

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from transformers_turboquant import apply_turboquant
from transformers_turboquant.base import TurboQuantAttentionBase
from transformers_turboquant.registry import UnsupportedModelError, get_attention_class, register_family
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2
from turboquant_pytorch.kernels import (asymmetric_attention_scores, lloyd_max_dequantize,
                                        lloyd_max_quantize, pack_bits, unpack_bits)

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------- reference golden vectors

@pytest.mark.parametrize("tag", ["d64_b3", "d128_b2", "d128_b4"])
def test_cpu_branch_matches_reference_vectors(tag):
    g = np.load(os.path.join(GOLDEN, "cpu_compress.npz"))
    d, bits = (int(s[1:]) for s in tag.split("_"))
    kc = TurboQuantCompressorV2(d, bits, seed=42, use_triton=False)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, use_triton=False)
    x = torch.from_numpy(g[f"{tag}_x"])
    ck = kc.compress(x)
    assert np.array_equal(ck["k_mse"].numpy(), g[f"{tag}_k_mse"])
    assert np.array_equal(ck["qjl_signs"].numpy(), g[f"{tag}_qjl_signs"])
    assert np.array_equal(ck["residual_norm"].numpy(), g[f"{tag}_residual_norm"])
    q = torch.from_numpy(g[f"{tag}_q"])
    assert np.allclose(kc.asymmetric_attention_scores(q, ck).numpy(), g[f"{tag}_scores"], rtol=1e-6, atol=1e-5)
    cv = vc.compress(torch.from_numpy(g[f"{tag}_v"]))
    assert np.array_equal(cv["indices"].numpy(), g[f"{tag}_v_indices"])
    assert np.array_equal(cv["vec_norms"].numpy(), g[f"{tag}_v_norms"])
    assert np.allclose(vc.decompress(cv).numpy(), g[f"{tag}_v_recon"], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("impl,fixture", [("eager", "gpt2_logits.npz"), ("sdpa", "gpt2_logits_sdpa.npz")])
def test_gpt2_config1_logits_match_reference(impl, fixture):
    """Config 1 with apply_turboquant's defaults: eager gets the decoder's additive causal
    mask, sdpa gets none and (as in the reference, gpt2.py:99-101) attends to every position."""
    from transformers import GPT2Config, GPT2LMHeadModel

    g = np.load(os.path.join(GOLDEN, fixture))
    torch.manual_seed(0)
    cfg = GPT2Config()
    cfg._attn_implementation = impl
    model = GPT2LMHeadModel(cfg).eval()
    assert apply_turboquant(model, bits=3, seed=42) is model
    with torch.no_grad():
        logits = model(input_ids=torch.from_numpy(g["input_ids"]).long()).logits[0]
    assert np.array_equal(logits[:8, :16].numpy(), g["logits_head"])
    assert np.array_equal(logits[-8:, -16:].numpy(), g["logits_tail"])
    assert np.allclose(logits.double().sum(-1).numpy(), g["row_sums"], rtol=0, atol=1e-6)
    assert np.array_equal(logits.argmax(-1).numpy(), g["argmax"])


# ---------------------------------------------------------------- CPU branch vs oracle

@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_cpu_compress_matches_oracle(bits, d):
    torch.manual_seed(0)
    x = torch.randn(1, 2, 16, d, dtype=torch.float16)
    kc = TurboQuantCompressorV2(d, bits, seed=42)
    ck = kc.compress(x)
    ref = O.key_compress_unpacked(x.numpy(), kc.Pi.numpy(), kc.S.numpy(), kc.centroids.numpy())
    assert (ck["qjl_signs"].numpy().reshape(-1, d) != ref["qjl_signs"]).mean() < 1e-3
    assert np.allclose(ck["k_mse"].numpy().reshape(-1, d).astype(np.float32),
                       ref["k_mse"].astype(np.float32), atol=2e-3)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042)
    cv = vc.compress(x)
    vref = O.value_compress_unpacked(x.numpy(), vc.Pi.numpy(), vc.centroids.numpy())
    assert (cv["indices"].numpy() != vref["indices"]).mean() < 1e-3


# ---------------------------------------------------------------- kernel functions on CPU

@pytest.mark.parametrize("b", [1, 2, 3, 4, 5, 6, 7, 8])
def test_cpu_pack_unpack_match_oracle(b):
    torch.manual_seed(42 + b)
    idx = torch.randint(0, 1 << b, (100, 128), dtype=torch.int32)
    packed = pack_bits(idx, b)
    assert packed.dtype == torch.uint8 and packed.shape == (100, math.ceil(128 * b / 8))
    assert np.array_equal(packed.numpy(), O.pack_bits(idx.numpy(), b))
    assert torch.equal(unpack_bits(packed, b, 128), idx)


def test_cpu_quantize_and_dequantize():
    torch.manual_seed(7)
    vc = TurboQuantCompressorMSE(128, 3, seed=0)
    y = torch.randn(100, 128) / math.sqrt(128)
    packed = lloyd_max_quantize(y, vc.boundaries, b_eff=3)
    codes = O.quantize_searchsorted(y.numpy(), vc.boundaries.numpy())
    assert np.array_equal(packed.numpy(), O.pack_bits(codes, 3))
    deq = lloyd_max_dequantize(packed, vc.centroids.half(), 3, 128)
    assert deq.dtype == torch.float16 and deq.shape == (100, 128)
    assert np.array_equal(deq.numpy(), O.dequantize(packed.numpy(), vc.centroids.numpy(), 3, 128))
    with pytest.raises(AssertionError):
        lloyd_max_quantize(y, vc.boundaries[:3], b_eff=3)


def test_cpu_asymmetric_scores_match_oracle():
    rng = np.random.default_rng(0)
    B, H, Sq, Sk, d, bits = 2, 4, 8, 16, 64, 3
    cent = torch.tensor([-0.2, -0.07, 0.07, 0.2]).half()
    codes = rng.integers(0, 4, size=(B * H * Sk, d))
    sb = rng.integers(0, 2, size=(B * H * Sk, d))
    q = torch.from_numpy(rng.standard_normal((B, H, Sq, d))).half()
    s_eff = torch.from_numpy(rng.standard_normal((d, d))).half()
    rn = torch.from_numpy(rng.random((B, H, Sk))).half()
    vn = torch.from_numpy(rng.random((B, H, Sk)) * 10).half()
    coeff = O.COEFF(d)
    out = asymmetric_attention_scores(
        q, torch.from_numpy(O.pack_bits(codes, 2)).view(B, H, Sk, -1),
        torch.from_numpy(O.pack_bits(sb, 1)).view(B, H, Sk, -1), rn,
        cent.unsqueeze(0).expand(H, -1), s_eff, vn, bits, coeff)
    assert out.dtype == torch.float32 and out.shape == (B, H, Sq, Sk)
    for bh in range(B * H):
        b_, h_ = divmod(bh, H)
        qr = q[b_, h_].numpy()
        qp = qr.astype(np.float64) @ s_eff.numpy().astype(np.float64).T
        ref = O.scores_packed(qr, qp, codes[bh * Sk:(bh + 1) * Sk], sb[bh * Sk:(bh + 1) * Sk],
                              rn[b_, h_].numpy(), vn[b_, h_].numpy(), cent.numpy(), coeff)
        assert O.rel_err(out[b_, h_].numpy(), ref) < 1e-5


# ---------------------------------------------------------------- byte accounting (reference test_memory.py)

@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_unpacked_bytes(bits, d):
    S = 64
    torch.manual_seed(0)
    x = torch.randn(1, 1, S, d, dtype=torch.float16)
    ck = TurboQuantCompressorV2(d, bits, seed=42, use_triton=False).compress(x)
    nbytes = sum(v.nbytes for v in ck.values() if isinstance(v, torch.Tensor))
    assert nbytes == S * (3 * d + 2)
    assert ck["k_mse"].dtype == torch.float16 and ck["qjl_signs"].dtype == torch.int8
    cv = TurboQuantCompressorMSE(d, bits, seed=42, use_triton=False).compress(x)
    assert sum(v.nbytes for v in cv.values() if isinstance(v, torch.Tensor)) == S * (d + 2)
    assert cv["indices"].dtype == torch.uint8
    # packed records (the GPU format): keys ceil(d(b-1)/8) + d/8 + 4, values ceil(db/8) + 2
    assert math.ceil(d * (bits - 1) / 8) + d // 8 + 4 < 2 * d
    assert math.ceil(d * bits / 8) + 2 < 2 * d


# ---------------------------------------------------------------- registry (reference test_registry.py)

def test_registry_dispatch_and_errors():
    @register_family("_test_a", "_test_b")
    class _Fake(TurboQuantAttentionBase):
        ATTENTION_CLASS_NAMES = ("_Fake",)

        @classmethod
        def from_original(cls, original, key_compressor, val_compressor):
            raise NotImplementedError

        def forward(self, hidden_states, **kwargs):
            raise NotImplementedError

    assert get_attention_class("_test_a") is _Fake and get_attention_class("_test_b") is _Fake
    with pytest.raises(UnsupportedModelError) as e:
        get_attention_class("__nonexistent_xyz__")
    msg = str(e.value)
    assert "__nonexistent_xyz__" in msg and "Supported:" in msg and "@register_family" in msg
    for mt in ("gpt2", "qwen2", "llama", "mistral", "deepseek"):
        assert issubclass(get_attention_class(mt), TurboQuantAttentionBase)


# ---------------------------------------------------------------- apply_turboquant on local random-init models

def _tiny_llama(model_type="llama"):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(0)
    if model_type == "qwen2":
        cfg = Qwen2Config(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                          num_attention_heads=4, num_key_value_heads=2)
        return Qwen2ForCausalLM(cfg).eval()
    cfg = LlamaConfig(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2)
    return LlamaForCausalLM(cfg).eval()


@pytest.mark.parametrize("model_type", ["llama", "qwen2"])
def test_apply_turboquant_llama_like(model_type):
    from transformers_turboquant.families.llama import TurboQuantLlamaAttention
    from transformers_turboquant.families.qwen2 import TurboQuantQwen2Attention

    model = _tiny_llama(model_type)
    cls = TurboQuantLlamaAttention if model_type == "llama" else TurboQuantQwen2Attention
    n_before = sum(type(m).__name__ in cls.ATTENTION_CLASS_NAMES for m in model.modules())
    assert apply_turboquant(model, bits=3) is model
    assert sum(isinstance(m, cls) for m in model.modules()) == n_before == 2
    assert model.config.use_cache is False
    ids = torch.randint(0, 128, (1, 12))
    with torch.no_grad():
        out = model.generate(ids, max_new_tokens=4, do_sample=False)
    assert out.shape == (1, 16)
    # layer seeds: seed+i for keys, seed+i+10000 for values (patch.py:62-75)
    layers = [m for m in model.modules() if isinstance(m, cls)]
    assert torch.equal(layers[1].key_compressor.Pi, TurboQuantCompressorV2(32, 3, seed=43).Pi)
    assert torch.equal(layers[0].val_compressor.Pi, TurboQuantCompressorMSE(32, 3, seed=10042).Pi)


def _small_gpt2(impl, **kw):
    from transformers import GPT2Config, GPT2LMHeadModel

    torch.manual_seed(0)
    cfg = GPT2Config(n_layer=2, n_embd=128, n_head=2, vocab_size=256)
    cfg._attn_implementation = impl
    return apply_turboquant(GPT2LMHeadModel(cfg).eval(), bits=3, seed=42, **kw)


def test_causal_auto_matches_explicit_mask():
    """causal='auto' under sdpa (no mask passed) equals eager with its additive causal mask."""
    ids = torch.arange(24).unsqueeze(0)
    with torch.no_grad():
        eager = _small_gpt2("eager")(input_ids=ids).logits
        auto = _small_gpt2("sdpa", causal="auto")(input_ids=ids).logits
    assert torch.allclose(eager, auto, atol=1e-5)


def test_default_is_reference_noncausal_under_sdpa():
    """The default adds a mask only when one is passed (gpt2.py:99-101): under sdpa every
    layer attends to all positions, i.e. each attention module equals itself fed an all-zero
    additive mask, and the logits differ from the causal eager run."""
    ids = torch.arange(24).unsqueeze(0)
    model = _small_gpt2("sdpa")
    attn = model.transformer.h[0].attn
    hidden = torch.randn(1, 24, 128, generator=torch.Generator().manual_seed(3))
    with torch.no_grad():
        none, _ = attn(hidden)
        zero, _ = attn(hidden, attention_mask=torch.zeros(1, 1, 24, 24))
        assert torch.equal(none, zero)
        assert not torch.allclose(model(input_ids=ids).logits, _small_gpt2("eager")(input_ids=ids).logits,
                                  atol=1e-3)
