"""Benchmark of the TurboQuant compressed-attention hot path on one MI355X.

Workload: one attention layer of Llama-3-8B shape,
batch 1, 32 query heads, 8 KV heads, head_dim 128, seq 8192, bf16 Q/K/V ~ N(0,1)
with 4 outlier channels x20 on K, bits=3.  A step = compress K and V (fused HIP
kernels), prepare queries, and causal compressed-domain attention for all 8192
query positions (scores + online softmax + P.V in one kernel).

Metric: compressed-attention key*heads/s (one key*head = one (query row, query
head, key) score evaluated; causal => B*Hq*S(S+1)/2 per step) plus compress
tokens/s.  Prints one JSON line.  With --gpus N > 1 it exits: this build runs on
one GPU.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "transformers-turboquant_amd"))

B, HQ, HKV, S, D, BITS = 1, 32, 8, 8192, 128, 3
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def key_rec_bytes(bits: int, d: int) -> int:
    return math.ceil(d * (bits - 1) / 8) + d // 8 + 4


def val_rec_bytes(bits: int, d: int) -> int:
    return math.ceil(d * bits / 8) + 2


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (profiles/traffic_config2.json), scaled by the copy-kernel
    calibration recorded there; None if no such measurement is committed."""
    path = os.path.join(ROOT, "profiles", "traffic_config2.json")
    try:
        with open(path) as f:
            rec = json.load(f)
        return rec["kernels"][kernel]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline(seconds_budget: float) -> dict:
    """The oracle (numpy restatement of the reference's PyTorch branch) on a bounded
    slice of the same workload: one KV head group (4 query heads), the first S_cpu
    positions, causal; compress + scores + softmax + P.V timed together."""
    import numpy as np
    import torch

    from oracle import tq_oracle as O
    from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

    s_cpu = S  # one KV-head group of the full 8192-token workload
    g = HQ // HKV
    rng = np.random.default_rng(0)
    k = rng.standard_normal((s_cpu, D)).astype(np.float32)
    k[:, :4] *= 20
    v = rng.standard_normal((s_cpu, D)).astype(np.float32)
    q = rng.standard_normal((g, s_cpu, D)).astype(np.float32)
    kc = TurboQuantCompressorV2(D, BITS, seed=42)
    vc = TurboQuantCompressorMSE(D, BITS, seed=10042)
    pi_k, s_k, ck_ = kc.Pi.numpy(), kc.S.numpy(), kc.centroids.numpy()
    pi_v, cv_ = vc.Pi.numpy(), vc.centroids.numpy()
    coeff = O.COEFF(D)

    def run():
        kk = O.key_compress_unpacked(k, pi_k, s_k, ck_)
        vv = O.value_compress_unpacked(v, pi_v, cv_)
        vals = O.value_decompress(vv["indices"], vv["vec_norms"], pi_v, cv_, dtype=np.float32)
        for h in range(g):
            sc = O.scores_unpacked(q[h], kk["k_mse"], kk["qjl_signs"], kk["residual_norm"], s_k, coeff,
                                   dtype=np.float32)
            O.attention(sc, vals, 1 / math.sqrt(D), causal=True, dtype=np.float32)

    run()  # warm-up
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 and time.perf_counter() - t_start < seconds_budget:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    key_heads = g * s_cpu * (s_cpu + 1) // 2
    try:
        from threadpoolctl import threadpool_info
        threads = max(int(i.get("num_threads", 1)) for i in threadpool_info()) if threadpool_info() else 1
    except Exception:  # pragma: no cover
        threads = os.cpu_count() or 1
    return {
        "value": key_heads / t,
        "unit": "key*heads/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle (numpy f32 restatement of the reference PyTorch branch) on 1 KV head x {g} query "
                   f"heads, {s_cpu} positions causal: compress K/V + scores + softmax + P.V; median of "
                   f"{len(times)} runs, {t * 1e3:.0f} ms/run; host {platform.processor() or platform.machine()}"),
    }


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=30.0)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run one device-to-device copy of MIB MiB first (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU runs are not part of it.", file=sys.stderr)
        sys.exit(2)

    import torch

    from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2
    from turboquant_pytorch.fused import attention_from_prepared

    dev = "cuda"
    gen = torch.Generator(device="cpu").manual_seed(0)
    q = torch.randn(B, HQ, S, D, generator=gen).to(dev, torch.bfloat16)
    k = torch.randn(B, HKV, S, D, generator=gen)
    outliers = torch.randperm(D, generator=torch.Generator().manual_seed(1))[:4]
    k[..., outliers] *= 20.0
    k = k.to(dev, torch.bfloat16)
    v = torch.randn(B, HKV, S, D, generator=gen).to(dev, torch.bfloat16)
    kc = TurboQuantCompressorV2(D, BITS, seed=42, device=dev)
    vc = TurboQuantCompressorMSE(D, BITS, seed=10042, device=dev)

    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    marks = []

    def step(record: bool):
        e = [ev() for _ in range(4)] if record else None
        if record:
            e[0].record()
        ck = kc.compress(k)
        cv = vc.compress(v)
        if record:
            e[1].record()
        q_rot, q_proj = kc.prepare_queries(q)
        if record:
            e[2].record()
        out = attention_from_prepared(q_rot, q_proj, kc, vc, ck, cv, causal=True, out_dtype=torch.bfloat16)
        if record:
            e[3].record()
            marks.append(e)
        return out

    for _ in range(args.warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step(True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    compress_ms = sum(m[0].elapsed_time(m[1]) for m in marks) / len(marks)
    prep_ms = sum(m[1].elapsed_time(m[2]) for m in marks) / len(marks)
    attn_ms = sum(m[2].elapsed_time(m[3]) for m in marks) / len(marks)
    ms_per_step = elapsed / args.steps * 1e3
    key_heads = B * HQ * S * (S + 1) // 2
    attn_flops = key_heads * (2 * D + 2 * D + 2 * D)  # term 1, QJL term, P.V
    tokens = B * S
    compress_bytes = B * HKV * S * (2 * D * 2 + key_rec_bytes(BITS, D) + val_rec_bytes(BITS, D))
    achieved_tflops = attn_flops / (attn_ms * 1e-3) / 1e12

    rec = {
        "metric": "compressed-attn keys*heads/s scored (causal prefill, config 2) + compress tokens/s",
        "value": key_heads / (ms_per_step * 1e-3),
        "unit": "key*heads/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16-mfma/f32-acc",
        "data": "synthetic (bf16 N(0,1) Q/K/V, 4 K channels x20, seed 0)",
        "config": {"workload": "configs[1]: Llama-3-8B attention layer, B1 Hq32 Hkv8 d128 S8192 bits3 causal",
                   "global_batch": B, "seq_len": S, "parallelism": "single-gpu"},
        "compress_tokens_per_s": tokens / (compress_ms * 1e-3),
        "compress_ms": compress_ms,
        "compress_hbm_gbs": compress_bytes / (compress_ms * 1e-3) / 1e9,
        "query_prep_ms": prep_ms,
        "attention_ms": attn_ms,
        "roofline": {
            "kernel": "tq::attn_kernel<128, 2, false, false> (fused scores + softmax + P.V)",
            "bound": "mfma",
            "achieved": achieved_tflops,
            "peak": MFMA_F16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved_tflops / MFMA_F16_PEAK_TFLOPS,
            "traffic": measured_traffic("attn_kernel"),
        },
    }
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
