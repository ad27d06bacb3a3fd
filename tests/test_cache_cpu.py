"""The compressed KV cache on the CPU path (reference semantics, unpacked format).

Decoding with a TurboQuantCache must give what the reference's cache-less
recomputation gives: cached positions are compressed once with the same
per-row arithmetic, so every step attends to the same codes.
"""

import pytest
import torch

from transformers_turboquant import TurboQuantCache, apply_turboquant
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2


def _model(kind):
    from transformers import GPT2Config, GPT2LMHeadModel, LlamaConfig, LlamaForCausalLM

    torch.manual_seed(0)
    if kind == "gpt2":
        cfg = GPT2Config(n_layer=2, n_embd=128, n_head=2, vocab_size=256)
        cfg._attn_implementation = "eager"
        return GPT2LMHeadModel(cfg).eval()
    cfg = LlamaConfig(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2)
    return LlamaForCausalLM(cfg).eval()


@pytest.mark.parametrize("kind", ["llama", "gpt2"])
def test_cached_generate_matches_recompute(kind):
    # decoding one token at a time is causal by construction, so the recomputation it is
    # compared with must be too: causal="auto" masks the prompt when the decoder passes no
    # mask (the default reproduces the reference, which then attends to every position)
    model = apply_turboquant(_model(kind), bits=3, seed=42, causal="auto")
    ids = torch.randint(0, 128, (2, 11), generator=torch.Generator().manual_seed(3))
    kw = dict(max_new_tokens=6, min_new_tokens=6, do_sample=False, output_scores=True,
              return_dict_in_generate=True, attention_mask=torch.ones_like(ids))
    with torch.no_grad():
        ref = model.generate(ids, use_cache=False, **kw)
        cache = TurboQuantCache()
        got = model.generate(ids, use_cache=True, past_key_values=cache, **kw)
    assert torch.equal(got.sequences, ref.sequences)
    for a, b in zip(got.scores, ref.scores):
        assert torch.allclose(a, b, rtol=1e-4, atol=1e-4)
    # the prompt and every generated token but the last were appended
    assert cache.get_seq_length() == ids.shape[1] + 5
    assert cache.nbytes() > 0


def test_cache_layer_append_crop_reorder():
    d, B, H = 32, 3, 2
    kc = TurboQuantCompressorV2(d, 3, seed=1)
    vc = TurboQuantCompressorMSE(d, 3, seed=10001)
    g = torch.Generator().manual_seed(0)
    k = torch.randn(B, H, 20, d, generator=g)
    v = torch.randn(B, H, 20, d, generator=g)
    cache = TurboQuantCache()
    cache.append(0, kc, vc, k[:, :, :13], v[:, :, :13])
    ck, cv = cache.append(0, kc, vc, k[:, :, 13:], v[:, :, 13:])
    full_k, full_v = kc.compress(k), vc.compress(v)
    for name in ("k_mse", "qjl_signs", "residual_norm"):
        assert torch.equal(ck[name], full_k[name]), name
    for name in ("indices", "vec_norms"):
        assert torch.equal(cv[name], full_v[name]), name
    assert cache.get_seq_length() == 20 and cache.get_mask_sizes(1, 0) == (21, 0)

    cache.crop(-4)
    lay = cache.layer(0)
    assert lay.get_seq_length() == 16
    assert torch.equal(lay.cpu_k["k_mse"], full_k["k_mse"][:, :, :16])
    assert torch.equal(lay.cpu_v["indices"], full_v["indices"].reshape(B, H, 20, d)[:, :, :16].reshape(-1, d))

    cache.reorder_cache(torch.tensor([2, 0, 2]))
    assert torch.equal(lay.cpu_k["qjl_signs"], full_k["qjl_signs"][[2, 0, 2], :, :16])
    assert torch.equal(lay.cpu_v["vec_norms"].reshape(3, H, 16),
                       full_v["vec_norms"].reshape(B, H, 20)[[2, 0, 2], :, :16])
    cache.reset()
    assert cache.get_seq_length() == 0


def test_cache_rejects_uncompressed_update():
    cache = TurboQuantCache()
    with pytest.raises(NotImplementedError):
        cache.update(torch.zeros(1, 1, 1, 8), torch.zeros(1, 1, 1, 8), 0)


def test_append_refuses_other_compressor_settings():
    """Positions compressed under one (bits, seed) pair must not be extended under another:
    the new compressor's Pi/S would then be applied to the old planes."""
    d = 32
    g = torch.Generator().manual_seed(1)
    k = torch.randn(1, 2, 5, d, generator=g)
    cache = TurboQuantCache()
    cache.append(0, TurboQuantCompressorV2(d, 3, seed=1), TurboQuantCompressorMSE(d, 3, seed=10001), k, k)
    with pytest.raises(ValueError, match="other settings"):
        cache.append(0, TurboQuantCompressorV2(d, 3, seed=2), TurboQuantCompressorMSE(d, 3, seed=10001), k, k)
    with pytest.raises(ValueError, match="other settings"):
        cache.append(0, TurboQuantCompressorV2(d, 3, seed=1), TurboQuantCompressorMSE(d, 2, seed=10001), k, k)
    # the same settings keep appending; after a reset any settings start a new sequence
    cache.append(0, TurboQuantCompressorV2(d, 3, seed=1), TurboQuantCompressorMSE(d, 3, seed=10001), k, k)
    assert cache.get_seq_length() == 10
    cache.layer(0).reset()
    cache.append(0, TurboQuantCompressorV2(d, 3, seed=2), TurboQuantCompressorMSE(d, 3, seed=10001), k, k)
