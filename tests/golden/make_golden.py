"""Write golden fixtures for the parts of the hot path that no closed form pins.

Run in the build container only (the reference is not present on GPU boxes):

    python tests/golden/make_golden.py /root/reference

It imports the reference's own CPU code (src/turboquant_pytorch/compressors.py
and src/transformers_turboquant) and records, as small JSON/NPZ data files:

  codebooks.json      exact f32 centroids of the compressors' Lloyd-Max solver
                      (compressors.py:72-96) for head_dim 32/64/128/256, bits 1-4
  setup.json          sha256 of Pi, S (keys) and Pi (values) for the seeds used by
                      the configs (compressors.py:50-70, patch.py:62-75)
  cpu_compress.npz    the PyTorch-branch compress dicts and scores of a seeded
                      input (compressors.py:139-161, :201-224, :288-317)
  gpt2_logits.npz     config 1 (GPT-2 small random init, bits=3 seed=42, 512
                      tokens) logits slice + checksum, eager attention

Everything else (bit layout, quantisation rule, estimator, softmax) is pinned by
closed forms in tests/test_oracle_pins.py.
"""

from __future__ import annotations

import hashlib
import json
import os
import sys
import warnings

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().cpu().contiguous().float().numpy().tobytes()).hexdigest()


def main(ref_root: str) -> None:
    sys.path.insert(0, os.path.join(ref_root, "src"))
    warnings.filterwarnings("ignore")
    from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

    # ---- codebooks
    books = {}
    for d in (32, 64, 128, 256):
        for bits in (1, 2, 3, 4):
            # V2 with bits+1 uses mse_bits = bits; MSE compressor uses bits directly
            comp = TurboQuantCompressorMSE(d, bits, seed=0)
            books[f"d{d}_b{bits}"] = {
                "centroids_hex": [float(x).hex() for x in comp.centroids.tolist()],
                "boundaries_hex": [float(x).hex() for x in comp.boundaries.tolist()],
            }
    with open(os.path.join(HERE, "codebooks.json"), "w") as f:
        json.dump(books, f, indent=1)

    # ---- seeded set-up: seed 0 and every per-layer seed the benchmark configurations use
    # (patch.py:62-75: layer i takes seed+i for keys, seed+i+10000 for values and the key S);
    # head_dim 64 covers GPT-2 small's 12 layers, head_dim 128 the 36 layers of Qwen2.5-3B
    # (Llama-3.1-8B's 32 and DeepSeek-7B's 30 are a prefix of them)
    setup = {}
    for d, seeds in ((64, [0] + list(range(42, 54))), (128, [0] + list(range(42, 78)))):
        for seed in seeds:
            kc = TurboQuantCompressorV2(d, 3, seed=seed)
            vc = TurboQuantCompressorMSE(d, 3, seed=seed + 10000)
            setup[f"d{d}_s{seed}"] = {
                "key_pi": sha(kc.Pi), "key_s": sha(kc.S), "val_pi": sha(vc.Pi),
                "key_pi_00": float(kc.Pi[0, 0]).hex(), "key_s_00": float(kc.S[0, 0]).hex(),
            }
    with open(os.path.join(HERE, "setup.json"), "w") as f:
        json.dump(setup, f, indent=1)

    # ---- the reference's rotations themselves for every per-layer seed of the benchmark
    # configurations (GPT-2 small's 12 layers at head_dim 64, Qwen2.5-3B's 36 at 128), as
    # the fallback a host whose LAPACK rounds the QR differently pins
    # (codebook.pin_rotations).  The MI355X boxes' MKL differs from this container's by
    # up to ~1e-6 per element, whatever its thread count or MKL_CBWR mode.
    rots = {}
    for d, seeds in ((64, range(42, 54)), (128, range(42, 78))):
        for seed in seeds:
            rots[f"d{d}_s{seed}"] = TurboQuantCompressorV2(d, 3, seed=seed).Pi.numpy()
            rots[f"d{d}_s{seed + 10000}"] = TurboQuantCompressorMSE(d, 3, seed=seed + 10000).Pi.numpy()
    np.savez_compressed(os.path.join(HERE, "rotations.npz"), **rots)

    # ---- CPU-branch compress / scores / decompress on a seeded input
    out = {}
    for d, bits in ((64, 3), (128, 2), (128, 4)):
        gen = torch.Generator().manual_seed(1234 + d + bits)
        x = torch.randn(1, 2, 16, d, generator=gen).to(torch.float16)
        v = torch.randn(1, 2, 16, d, generator=gen).to(torch.float16)
        q = torch.randn(1, 2, 8, d, generator=gen).to(torch.float16)
        kc = TurboQuantCompressorV2(d, bits, seed=42, use_triton=False)
        vc = TurboQuantCompressorMSE(d, bits, seed=10042, use_triton=False)
        ck = kc.compress(x)
        cv = vc.compress(v)
        tag = f"d{d}_b{bits}"
        out[f"{tag}_x"] = x.numpy()
        out[f"{tag}_v"] = v.numpy()
        out[f"{tag}_q"] = q.numpy()
        out[f"{tag}_k_mse"] = ck["k_mse"].numpy()
        out[f"{tag}_qjl_signs"] = ck["qjl_signs"].numpy()
        out[f"{tag}_residual_norm"] = ck["residual_norm"].numpy()
        out[f"{tag}_scores"] = kc.asymmetric_attention_scores(q, ck).numpy()
        out[f"{tag}_v_indices"] = cv["indices"].numpy()
        out[f"{tag}_v_norms"] = cv["vec_norms"].numpy()
        out[f"{tag}_v_recon"] = vc.decompress(cv).numpy()
    np.savez_compressed(os.path.join(HERE, "cpu_compress.npz"), **out)

    # ---- config 1: GPT-2 small random init under both attention implementations. eager
    # passes an additive causal mask; sdpa passes none, so the wrapper (gpt2.py:99-101)
    # attends to every position.
    from transformers import GPT2Config, GPT2LMHeadModel
    from transformers_turboquant import apply_turboquant

    for impl, name in (("eager", "gpt2_logits.npz"), ("sdpa", "gpt2_logits_sdpa.npz")):
        torch.manual_seed(0)
        cfg = GPT2Config()
        cfg._attn_implementation = impl
        model = GPT2LMHeadModel(cfg).eval()
        apply_turboquant(model, bits=3, seed=42)
        ids = torch.randint(0, 50257, (1, 512), generator=torch.Generator().manual_seed(0))
        with torch.no_grad():
            logits = model(input_ids=ids).logits
        np.savez_compressed(
            os.path.join(HERE, name),
            input_ids=ids.numpy().astype(np.int32),
            logits_head=logits[0, :8, :16].numpy(),
            logits_tail=logits[0, -8:, -16:].numpy(),
            row_sums=logits[0].double().sum(-1).numpy(),
            argmax=logits[0].argmax(-1).numpy().astype(np.int32),
        )
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
