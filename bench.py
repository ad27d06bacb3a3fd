"""Benchmark of the TurboQuant compressed-attention hot path on one MI355X.

Workload: one attention layer of Llama-3-8B shape,
32 query heads, 8 KV heads (GQA group 4), head_dim 128, bf16 Q/K/V ~ N(0,1)
with 4 outlier channels x20 on K, bits=3.

Headline (`value`, HBM roofline): decode-shaped compressed-key scoring at 32k
context, the regime the metric's "% of HBM peak" refers to.  A step is one
tq_attention_scores launch scoring one query row of each of DEC_B sequences
against its 32768 compressed keys (all 32 query heads; materialised f32
scores, the reference's scoring API).  Steps rotate over DEC_ROT distinct
caches so the working set (>1 GB) is far beyond the 256 MB MALL.  The same
shape is also timed through the fused decode attention (softmax . V).

Secondary legs in the same line: compress tokens/s and the causal prefill of
8192 positions (scores + online softmax + P.V for every query row, MFMA
roofline).  Prints one JSON line.  With --gpus N > 1 it exits: this build runs
on one GPU.
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
DEC_B, DEC_SK, DEC_ROT = 16, 32768, 4
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def key_rec_bytes(bits: int, d: int) -> int:
    return math.ceil(d * (bits - 1) / 8) + d // 8 + 4


def val_rec_bytes(bits: int, d: int) -> int:
    return math.ceil(d * bits / 8) + 2


def measured_traffic(kernel: str, record: str = "traffic_bench.json"):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE passes (profiles/<record>), scaled by the copy-kernel calibration
    recorded there; None if no such measurement is committed."""
    path = os.path.join(ROOT, "profiles", record)
    try:
        with open(path) as f:
            rec = json.load(f)
        return rec["kernels"][kernel]["traffic_bytes"]
    except (OSError, KeyError, ValueError):
        return None


def cpu_baseline_decode(seconds_budget: float) -> dict:
    """The oracle's f32 restatement of the reference's PyTorch scoring branch
    (compressors.py:201-224: q.k_mse^T + coeff * (q S^T).signs^T * rn) on a bounded
    sample of the decode workload: one query row of 4 query heads against the
    32768 keys of one KV head, repeated until the time budget is spent."""
    import numpy as np

    from oracle import tq_oracle as O
    from turboquant_pytorch.compressors import TurboQuantCompressorV2

    g = HQ // HKV
    rng = np.random.default_rng(0)
    kc = TurboQuantCompressorV2(D, BITS, seed=42)
    k = rng.standard_normal((DEC_SK, D)).astype(np.float32)
    k[:, :4] *= 20
    kk = O.key_compress_unpacked(k, kc.Pi.numpy(), kc.S.numpy(), kc.centroids.numpy())
    q = rng.standard_normal((g, 1, D)).astype(np.float32)
    s_mat, coeff = kc.S.numpy(), O.COEFF(D)

    def run():
        for h in range(g):
            O.scores_unpacked(q[h], kk["k_mse"], kk["qjl_signs"], kk["residual_norm"], s_mat, coeff,
                              dtype=np.float32)

    run()
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds_budget or n < 3:
        run()
        n += 1
    t = (time.perf_counter() - t0) / n
    return {
        "value": g * DEC_SK / t,
        "unit": "key*heads/s",
        "cores": _blas_threads(),
        "kind": "port",
        "sample": (f"oracle f32 scoring (reference PyTorch branch restated) of 1 query row x {g} query heads "
                   f"against one KV head's {DEC_SK} compressed keys, {n} repetitions in {n * t:.1f} s "
                   f"({t * 1e3:.1f} ms each); host {platform.processor() or platform.machine()}"),
    }


def _blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info
        info = threadpool_info()
        return max(int(i.get("num_threads", 1)) for i in info) if info else 1
    except Exception:  # pragma: no cover
        return os.cpu_count() or 1


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
    return {
        "value": key_heads / t,
        "unit": "key*heads/s",
        "cores": _blas_threads(),
        "kind": "port",
        "sample": (f"oracle (numpy f32 restatement of the reference PyTorch branch) on 1 KV head x {g} query "
                   f"heads, {s_cpu} positions causal: compress K/V + scores + softmax + P.V; median of "
                   f"{len(times)} runs, {t * 1e3:.0f} ms/run; host {platform.processor() or platform.machine()}"),
    }


def _events(n):
    import torch
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def decode_legs(kc, vc, outliers, steps: int, warmup: int) -> tuple[dict, dict]:
    """Decode-shaped scoring (the headline) and fused decode attention.

    DEC_ROT caches of DEC_B sequences x HKV heads x DEC_SK keys are compressed
    once; launch i uses cache i % DEC_ROT.  The C entry points are called
    directly with preallocated outputs so that launches queue back to back on
    torch's current stream, and HIP events on that stream bracket the timed
    launches.
    """
    import torch

    from turboquant_pytorch import _native
    from turboquant_pytorch.compressors import _tables

    dev = "cuda"
    lib = _native.lib()
    gen = torch.Generator(device=dev).manual_seed(2)
    caches = []
    for _ in range(DEC_ROT):
        k = torch.randn(DEC_B, HKV, DEC_SK, D, device=dev, generator=gen).to(torch.bfloat16)
        k[..., outliers.to(dev)] *= 20.0
        ck = kc.compress(k)
        del k
        v = torch.randn(DEC_B, HKV, DEC_SK, D, device=dev, generator=gen).to(torch.bfloat16)
        cv = vc.compress(v)
        del v
        caches.append((ck, cv))
    q = torch.randn(DEC_B, HQ, 1, D, device=dev, generator=gen).to(torch.bfloat16)
    q_rot, q_proj = kc.prepare_queries(q)
    tk = _tables(kc, dev, with_qjl=True)
    tv = _tables(vc, dev, with_qjl=False)
    coeff = math.sqrt(math.pi / 2) / D
    stream = torch.cuda.current_stream().cuda_stream
    scores = [torch.empty(DEC_B, HQ, 1, DEC_SK, dtype=torch.float32, device=dev) for _ in range(DEC_ROT)]
    outs = [torch.empty(DEC_B, 1, HQ, D, dtype=torch.bfloat16, device=dev) for _ in range(DEC_ROT)]
    ws_bytes = lib.tq_attention_workspace_size(DEC_B, HQ, HKV, 1, DEC_SK, D, BITS)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)

    def launch_scores(i):
        ck, _ = caches[i % DEC_ROT]
        return lib.tq_attention_scores(
            q_rot.data_ptr(), q_proj.data_ptr(), ck["packed_key_indices"].data_ptr(),
            ck["packed_qjl_signs"].data_ptr(), ck["residual_norm"].data_ptr(), ck["vec_norms"].data_ptr(),
            tk.cent16.data_ptr(), DEC_B, HQ, HKV, 1, DEC_SK, D, BITS, coeff,
            scores[i % DEC_ROT].data_ptr(), stream)

    def launch_attn(i):
        ck, cv = caches[i % DEC_ROT]
        o = outs[i % DEC_ROT]
        return lib.tq_attention_fwd(
            q_rot.data_ptr(), q_proj.data_ptr(), ck["packed_key_indices"].data_ptr(),
            ck["packed_qjl_signs"].data_ptr(), ck["residual_norm"].data_ptr(), ck["vec_norms"].data_ptr(),
            tk.cent16.data_ptr(), BITS, cv["packed_indices"].data_ptr(), cv["vec_norms"].data_ptr(),
            tv.cent32.data_ptr(), BITS, tv.pit_split.data_ptr(), DEC_B, HQ, HKV, 1, DEC_SK, D, coeff,
            1.0 / math.sqrt(D), 1, None, 0, 0, 0, 0, o.data_ptr(), _native.TQ_BF16,
            o.stride(0), o.stride(2), o.stride(1), ws.data_ptr(), ws_bytes, stream)

    def timed(launch):
        for i in range(warmup):
            _native.check(launch(i), "decode warmup")
        torch.cuda.synchronize()
        e0, e1 = _events(2)
        e0.record()
        for i in range(steps):
            st = launch(i)
            if st:
                _native.check(st, "decode launch")
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    ms_scores = timed(launch_scores)
    ms_attn = timed(launch_attn)
    key_heads = DEC_B * HQ * DEC_SK
    q_bytes = DEC_B * HQ * D * 2 * 2
    score_bytes = DEC_B * HKV * DEC_SK * key_rec_bytes(BITS, D) + key_heads * 4 + q_bytes
    attn_bytes = (DEC_B * HKV * DEC_SK * (key_rec_bytes(BITS, D) + val_rec_bytes(BITS, D)) + q_bytes
                  + DEC_B * HQ * D * 2)
    gbs_s = score_bytes / (ms_scores * 1e-3) / 1e9
    gbs_a = attn_bytes / (ms_attn * 1e-3) / 1e9
    scores_leg = {
        "ms_per_launch": ms_scores,
        "key_heads_per_s": key_heads / (ms_scores * 1e-3),
        "roofline": {
            "kernel": "tq::decode_scores_kernel<128, 3, 3, 32> (scores, f32 written)",
            "bound": "hbm", "achieved": gbs_s, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": gbs_s / HBM_PEAK_GBS, "traffic": measured_traffic("tq::decode_scores_kernel<128, 3, 3, 32>"),
            "algorithmic_bytes_per_launch": score_bytes,
        },
    }
    attn_leg = {
        "workload": f"fused decode attention, same caches: B{DEC_B} Hq{HQ} Hkv{HKV} Sq1 Sk{DEC_SK} bits{BITS}",
        "ms_per_launch": ms_attn,
        "key_heads_per_s": key_heads / (ms_attn * 1e-3),
        "roofline": {
            "kernel": "tq::decode_attn_lds_kernel<128, 3, 2, 2, false> + tq::decode_merge_kernel<128>",
            "bound": "hbm", "achieved": gbs_a, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": gbs_a / HBM_PEAK_GBS, "traffic": measured_traffic("decode_attention (attention + merge)"),
            "algorithmic_bytes_per_launch": attn_bytes,
        },
    }
    del caches, scores, outs, ws
    torch.cuda.empty_cache()
    return scores_leg, attn_leg


def prefill_leg(kc, vc, q, k, v, steps: int, warmup: int) -> dict:
    """Config-2 step: compress K and V, prepare queries, causal fused attention over
    all S query rows."""
    import torch

    from turboquant_pytorch.fused import attention_from_prepared

    marks = []

    def step(record: bool):
        e = _events(4) if record else None
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

    for _ in range(warmup):
        step(False)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    compress_ms = sum(m[0].elapsed_time(m[1]) for m in marks) / len(marks)
    prep_ms = sum(m[1].elapsed_time(m[2]) for m in marks) / len(marks)
    attn_ms = sum(m[2].elapsed_time(m[3]) for m in marks) / len(marks)
    ms_per_step = elapsed / steps * 1e3
    key_heads = B * HQ * S * (S + 1) // 2
    attn_flops = key_heads * (2 * D + 2 * D + 2 * D)  # term 1, QJL term, P.V
    compress_bytes = B * HKV * S * (2 * D * 2 + key_rec_bytes(BITS, D) + val_rec_bytes(BITS, D))
    tflops = attn_flops / (attn_ms * 1e-3) / 1e12
    return {
        "workload": f"causal prefill B{B} Hq{HQ} Hkv{HKV} d{D} S{S} bits{BITS}: compress K/V + query prep + "
                    "fused scores/softmax/P.V",
        "ms_per_step": ms_per_step,
        "key_heads_per_s": key_heads / (ms_per_step * 1e-3),
        "compress_tokens_per_s": B * S / (compress_ms * 1e-3),
        "compress_ms": compress_ms,
        "compress_hbm_gbs": compress_bytes / (compress_ms * 1e-3) / 1e9,
        "query_prep_ms": prep_ms,
        "attention_ms": attn_ms,
        "roofline": {
            "kernel": "tq::prefill_kernel<3, false> (fused scores + softmax + P.V)",
            "bound": "mfma", "achieved": tflops, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / MFMA_F16_PEAK_TFLOPS, "traffic": measured_traffic("tq::prefill_kernel<3, false>"),
        },
    }


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--no-prefill", action="store_true", help="skip the causal prefill / compress leg")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run one device-to-device copy of MIB MiB first (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); "
              "multi-GPU runs are not part of it.", file=sys.stderr)
        sys.exit(2)

    import torch

    from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

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

    scores_leg, attn_leg = decode_legs(kc, vc, outliers, args.steps, args.warmup)
    prefill = None if args.no_prefill else prefill_leg(kc, vc, q, k, v, args.steps, args.warmup)

    rec = {
        "metric": "compressed-attn keys*heads/s scored (% of HBM peak) + compress tokens/s",
        "value": scores_leg["key_heads_per_s"],
        "unit": "key*heads/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": scores_leg["ms_per_launch"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16-mfma/f32-acc",
        "data": "synthetic (bf16 N(0,1) Q/K/V, 4 K channels x20 = randperm(128, seed 1)[:4]; seeds 0 and 2)",
        "config": {"workload": (f"configs[1] Llama-3-8B attention (Hq{HQ} Hkv{HKV} d{D} bits{BITS}), decode-shaped "
                                f"scoring: 1 query row x {DEC_B} sequences x {DEC_SK} keys per step, rotating over "
                                f"{DEC_ROT} caches"),
                   "global_batch": DEC_B, "seq_len": DEC_SK, "parallelism": "single-gpu"},
        "roofline": scores_leg["roofline"],
        "compress_tokens_per_s": None if prefill is None else prefill["compress_tokens_per_s"],
        "decode_attention": attn_leg,
        "prefill": prefill,
    }
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline_decode(args.cpu_seconds / 2)
        if prefill is not None:
            prefill["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
