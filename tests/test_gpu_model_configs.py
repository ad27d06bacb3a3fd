"""Whole-model forwards at the benchmark configurations' scale (BASELINE.json configs[2..4]).

The reference path is one family forward() per layer (families/qwen2.py:69-125,
llama.py:18-122): q/k/v projections, rotary, compress K and V, asymmetric
scores, softmax, P.V over decompressed values, o_proj.  Each test builds the
random-init model on the GPU in bf16, patches it with apply_turboquant (the
reference's defaults: causal=False, seeds 42 + i / 42 + i + 10000), runs one
full-sequence forward with logits_to_keep=1, and checks

  * the logits are finite;
  * for the first and last layer, the module's output equals o_proj of the fused
    kernel on its own q / k / v (recomputed from the captured inputs), and that
    kernel output matches the float64 oracle on the device's packed planes
    (reference attention.py:419-461, compressors.py:186-189, qwen2.py:110-117)
    on sampled rows, within rel-err 1e-3 and cosine 0.9999.

  configs[2]  Qwen2.5-3B: 36 layers, hidden 2048, 16 / 2 heads, 4096 and 8192 tokens, bits 2 / 4
  configs[3]  Llama-3.1-8B: 32 layers, hidden 4096, 32 / 8 heads, 4 x 32768 tokens, bits 4
  configs[4]  DeepSeek-LLM-7B (model_type llama, MHA 32 / 32): 30 layers, 8 x 16384 tokens, bits 2
"""

import gc

import pytest
import torch

from test_gpu_configs import _check_rows
from turboquant_pytorch import compressed_attention

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(**kw):
    print("case:", kw, flush=True)


def _forward_and_check(model, cfg, B, S, bits, hq, hkv, d, rows_of):
    from transformers_turboquant import apply_turboquant

    model = model.to(torch.bfloat16).eval()
    apply_turboquant(model, bits=bits, seed=42)
    layers = model.model.layers
    last = len(layers) - 1
    captured = {}

    def hook(i):
        def fn(mod, args, kwargs, output):
            hs = kwargs["hidden_states"] if "hidden_states" in kwargs else args[0]
            captured[i] = (hs.detach(), kwargs["position_embeddings"], output[0].detach())
        return fn

    handles = [layers[i].self_attn.register_forward_hook(hook(i), with_kwargs=True) for i in (0, last)]
    ids = torch.randint(0, cfg.vocab_size, (B, S), generator=torch.Generator().manual_seed(S + bits)).to(DEV)
    with torch.no_grad():
        logits = model(input_ids=ids, logits_to_keep=1).logits
    torch.cuda.synchronize()
    for h in handles:
        h.remove()
    assert logits.shape == (B, 1, cfg.vocab_size) and torch.isfinite(logits).all()
    print(f"forward done: {len(layers)} layers, logits {tuple(logits.shape)}", flush=True)
    del logits
    for i in (0, last):
        hs, (cos, sin), mod_out = captured.pop(i)
        attn = layers[i].self_attn
        with torch.no_grad():
            q = attn.q_proj(hs).view(B, S, hq, d).transpose(1, 2)
            k = attn.k_proj(hs).view(B, S, hkv, d).transpose(1, 2)
            v = attn.v_proj(hs).view(B, S, hkv, d).transpose(1, 2)
            q, k = type(attn).apply_rotary(q, k, cos, sin)
            kc, vc = attn.key_compressor, attn.val_compressor
            ck, cv = kc.compress(k), vc.compress(v)
            del k, v
            out = compressed_attention(q, kc, vc, ck, cv, out_dtype=torch.float32)
            again = attn.o_proj(out.to(torch.bfloat16).reshape(B, S, -1))
        assert torch.equal(again, mod_out), i
        del again, mod_out
        picks = [(b, h, rows_of(S)) for b in sorted({0, B - 1}) for h in sorted({0, hq // 2 + 1, hq - 1})]
        _check_rows(out, q, kc, vc, ck, cv, hkv, picks, causal=False)
        del q, ck, cv, out
    gc.collect()
    torch.cuda.empty_cache()


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("S", [4096, 8192])
def test_qwen25_3b_model(S, bits):
    _case(config=2, S=S, bits=bits)
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=151936, hidden_size=2048, intermediate_size=11008, num_hidden_layers=36,
                      num_attention_heads=16, num_key_value_heads=2, max_position_embeddings=32768,
                      tie_word_embeddings=True)
    torch.manual_seed(0)
    with torch.device(DEV):
        model = Qwen2ForCausalLM(cfg)
    _forward_and_check(model, cfg, 1, S, bits, 16, 2, 128, lambda S: [0, 1, S // 2, S - 1])
    del model
    gc.collect()
    torch.cuda.empty_cache()


def test_llama31_8b_model_4x32768():
    _case(config=3, B=4, S=32768, bits=4)
    from transformers import LlamaConfig, LlamaForCausalLM

    cfg = LlamaConfig(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                      num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=131072,
                      rope_theta=500000.0)
    torch.manual_seed(0)
    with torch.device(DEV):
        model = LlamaForCausalLM(cfg)
    _forward_and_check(model, cfg, 4, 32768, 4, 32, 8, 128, lambda S: [0, S // 2, S - 1])
    del model
    gc.collect()
    torch.cuda.empty_cache()


def test_deepseek_llm_7b_model_8x16384():
    _case(config=4, B=8, S=16384, bits=2)
    from transformers import LlamaConfig, LlamaForCausalLM

    # DeepSeek-LLM-7B: model_type llama, 30 layers, MHA (32 query = 32 kv heads), vocab 102400
    cfg = LlamaConfig(vocab_size=102400, hidden_size=4096, intermediate_size=11008, num_hidden_layers=30,
                      num_attention_heads=32, num_key_value_heads=32, max_position_embeddings=16384)
    torch.manual_seed(0)
    with torch.device(DEV):
        model = LlamaForCausalLM(cfg)
    _forward_and_check(model, cfg, 8, 16384, 2, 32, 32, 128, lambda S: [0, S // 2, S - 1])
    del model
    gc.collect()
    torch.cuda.empty_cache()
