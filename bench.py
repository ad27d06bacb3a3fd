"""Benchmark of the TurboQuant compressed-attention hot path on one MI355X.

Headline (`value`, HBM roofline): the north-star target, compressed-key scoring
of Llama-3-8B-shaped attention (32 query heads, 8 KV heads, head_dim 128,
bits 3) at 32k context, decode-shaped (keys streamed once per query step: the
regime the metric's "% of HBM peak" refers to).  A step is one
tq_attention_scores launch scoring one query row of each of DEC_B sequences
against its 32768 compressed keys (all 32 query heads; materialised f32 scores,
the reference's scoring API).  Steps rotate over DEC_ROT distinct caches so the
working set (>1 GB) is far beyond the 256 MB MALL.  The same shape is also timed
through the fused decode attention (softmax . V).

Secondary legs in the same line: BASELINE.json configs[1] (the same layer shape
at 8192 tokens, bf16 Q/K/V ~ N(0,1) with 4 outlier channels x20 on K): compress
tokens/s and the causal prefill (scores + online softmax + P.V for every query
row, MFMA roofline); and one layer's eager decode step through the product path
(torch.ops.tq) at B = 1 with 4096 cached tokens, host and device time.  CPU
baselines: the build's torch CPU branch of the reference's PyTorch path on
bounded samples.  Prints one JSON line.  With --gpus N > 1 it exits: this build
runs on one GPU.
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
# the engine clock ramps from ~2.2 to ~2.4 GHz over the first ~50 ms of sustained load
# (constant GRBM_GUI_ACTIVE cycles per launch while the launch time falls 126 -> 115 us on
# the decode attention kernel); each decode leg runs this long untimed before its W
# warmup + K timed steps, so the timed steps see the clock a serving loop runs at
SETTLE_MS = 200.0
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


def host_cpu() -> dict:
    """The host the CPU baselines ran on: model name (from /proc/cpuinfo, as lscpu prints it),
    logical CPUs visible to this process, and torch's intra-op thread count."""
    import torch

    model = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    cpus = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"model": model, "logical_cpus": cpus, "torch_threads": torch.get_num_threads()}


def _cpu_threads() -> None:
    import torch

    cpus = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(max(1, cpus))


def cpu_baseline_decode(seconds_budget: float) -> dict:
    """The reference's PyTorch CPU branch as this build restates it (TurboQuantCompressorV2 on CPU
    tensors: compressors.py:139-161 compress, :201-224 scores; bit-exact with the reference's own
    outputs, tests/golden/cpu_compress.npz) on a bounded sample of the decode workload: one query
    row of the 4 query heads of one KV head against its 32768 compressed keys, repeated until the
    time budget is spent.  The keys are compressed once, untimed, as the GPU leg's caches are."""
    import torch

    from turboquant_pytorch.compressors import TurboQuantCompressorV2

    _cpu_threads()
    g = HQ // HKV
    gen = torch.Generator().manual_seed(0)
    kc = TurboQuantCompressorV2(D, BITS, seed=42)
    k = torch.randn(1, 1, DEC_SK, D, generator=gen)
    k[..., :4] *= 20
    ck = kc.compress(k.to(torch.bfloat16))
    q = torch.randn(1, g, 1, D, generator=gen).to(torch.bfloat16)
    kc.asymmetric_attention_scores(q, ck)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds_budget or n < 3:
        kc.asymmetric_attention_scores(q, ck)
        n += 1
    t = (time.perf_counter() - t0) / n
    host = host_cpu()
    return {
        "value": g * DEC_SK / t,
        "unit": "key*heads/s",
        "cores": host["torch_threads"],
        "kind": "port",
        "host": host,
        "sample": (f"torch CPU branch (reference PyTorch scoring restated, golden-pinned): 1 query row x {g} query "
                   f"heads against one KV head's {DEC_SK} compressed keys, {n} repetitions in {n * t:.1f} s "
                   f"({t * 1e3:.2f} ms each), {host['torch_threads']} threads on {host['model']}"),
    }


def cpu_baseline(seconds_budget: float) -> dict:
    """The same torch CPU branch on a bounded slice of the prefill workload: one KV head group
    (4 query heads) of the 8192-position causal layer, the reference's whole tail (families/
    qwen2.py:100-117): compress K and V, scores, /sqrt(d) + causal mask, softmax, decompress V,
    P.V; median of up to 3 runs after one warm-up."""
    import torch
    import torch.nn.functional as F

    from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

    _cpu_threads()
    g = HQ // HKV
    gen = torch.Generator().manual_seed(0)
    k = torch.randn(1, 1, S, D, generator=gen)
    k[..., :4] *= 20
    k = k.to(torch.bfloat16).repeat_interleave(g, dim=1)  # the reference expands K/V per query head
    v = torch.randn(1, 1, S, D, generator=gen).to(torch.bfloat16).repeat_interleave(g, dim=1)
    q = torch.randn(1, g, S, D, generator=gen).to(torch.bfloat16)
    kc = TurboQuantCompressorV2(D, BITS, seed=42)
    vc = TurboQuantCompressorMSE(D, BITS, seed=10042)
    causal = torch.full((S, S), float("-inf")).triu(1)

    def run():
        scores = kc.asymmetric_attention_scores(q, kc.compress(k)) / math.sqrt(D) + causal
        w = F.softmax(scores.float(), dim=-1).to(q.dtype)
        return torch.matmul(w, vc.decompress(vc.compress(v)).to(q.dtype))

    run()
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 and time.perf_counter() - t_start < seconds_budget:
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    t = sorted(times)[len(times) // 2]
    key_heads = g * S * (S + 1) // 2
    host = host_cpu()
    return {
        "value": key_heads / t,
        "unit": "key*heads/s",
        "cores": host["torch_threads"],
        "kind": "port",
        "host": host,
        "sample": (f"torch CPU branch on 1 KV head x {g} query heads, {S} positions causal: compress K/V + scores + "
                   f"softmax + P.V; median of {len(times)} runs, {t * 1e3:.0f} ms/run, "
                   f"{host['torch_threads']} threads on {host['model']}"),
    }


def _events(n):
    import torch
    return [torch.cuda.Event(enable_timing=True) for _ in range(n)]


def settle_clock(launch, ms: float = SETTLE_MS) -> int:
    """Launch back to back, untimed, until `ms` of GPU time has passed; returns the launch count."""
    import torch

    from turboquant_pytorch import _native

    n, spent = 0, 0.0
    while spent < ms:
        e0, e1 = _events(2)
        e0.record()
        for _ in range(16):
            _native.check(launch(n), "clock settle")
            n += 1
        e1.record()
        torch.cuda.synchronize()
        spent += e0.elapsed_time(e1)
    return n


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
        settle_clock(launch)
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
            "kernel": "tq::decode_scores_i8_kernel<2, 3> (scores, f32 written)",
            "bound": "hbm", "achieved": gbs_s, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": gbs_s / HBM_PEAK_GBS, "traffic": measured_traffic("tq::decode_scores_i8_kernel<2, 3>"),
            "algorithmic_bytes_per_launch": score_bytes,
        },
    }
    attn_leg = {
        "workload": f"fused decode attention, same caches: B{DEC_B} Hq{HQ} Hkv{HKV} Sq1 Sk{DEC_SK} bits{BITS}",
        "ms_per_launch": ms_attn,
        "key_heads_per_s": key_heads / (ms_attn * 1e-3),
        "roofline": {
            "kernel": "tq::decode_attn_i8_kernel<2, 2> + tq::decode_merge_kernel<128>",
            "bound": "hbm", "achieved": gbs_a, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": gbs_a / HBM_PEAK_GBS, "traffic": measured_traffic("decode_attention (attention + merge)"),
            "algorithmic_bytes_per_launch": attn_bytes,
        },
    }
    del caches, scores, outs, ws
    torch.cuda.empty_cache()
    return scores_leg, attn_leg


def compress_leg(kc, vc, steps: int, warmup: int) -> dict:
    """Compression at the north-star scale: keys and values of 4 sequences x 8 kv heads x 32768
    tokens (1,048,576 rows each, bf16, bits 3), timed separately with HIP events.  HBM: 256 B read
    + the record written per row (52 B keys, 50 B values).  MFMA: the f32-grade products run as
    f16 passes: a bf16 row is exact in f16 under a power-of-two row scale, so x Pi^T takes the
    weight's hi and lo parts (2 passes of d^2 MACs), while proj = u S_eff^T on the rotated-domain
    residual u takes hi.hi + lo.hi + hi.lo (3): keys 5 passes, values 2 -- the executed MFMA work,
    priced against the dense f16 peak."""
    import torch

    dev = "cuda"
    shape = (4, HKV, 32768, D)
    g = torch.Generator(device=dev).manual_seed(9)
    x = torch.randn(*shape, device=dev, generator=g).to(torch.bfloat16)
    rows = x.numel() // D
    out = {}
    for name, fn, rec, passes in (("keys", kc.compress, key_rec_bytes(BITS, D), 5),
                                  ("values", vc.compress, val_rec_bytes(BITS, D), 2)):
        for _ in range(warmup):
            fn(x)
        torch.cuda.synchronize()
        e0, e1 = _events(2)
        e0.record()
        for _ in range(steps):
            fn(x)
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / steps * 1e3
        gbs = rows * (2 * D + rec) / (us * 1e-6) / 1e9
        tflops = rows * passes * 2 * D * D / (us * 1e-6) / 1e12
        out[name] = {"us_per_launch": us, "rows_per_s": rows / (us * 1e-6), "hbm_gbs": gbs,
                     "hbm_frac": gbs / HBM_PEAK_GBS, "mfma_tflops": tflops,
                     "mfma_frac": tflops / MFMA_F16_PEAK_TFLOPS}
    both = out["keys"]["us_per_launch"] + out["values"]["us_per_launch"]
    return {"workload": f"B4 Hkv{HKV} S32768 d{D} bf16 bits{BITS}: {rows} key rows + {rows} value rows",
            "tokens_per_s": 4 * 32768 / (both * 1e-6), **out}


def decode_step_leg(kc, vc, cached: int = 4096, steps: int = 200) -> dict:
    """One attention layer's eager decode step through the product path (torch.ops.tq): compress the
    new token's K and V (8 kv heads), prepare the 32 query heads' query, split-K attention over the
    cached planes.  B = 1, bits 3.  Host time per step (wall clock over `steps` back-to-back steps,
    synchronised at the end) against device time (HIP events around the same steps)."""
    import torch

    from turboquant_pytorch import compressed_attention

    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(5)
    ck = kc.compress(torch.randn(1, HKV, cached, D, device=dev, generator=g).to(torch.bfloat16))
    cv = vc.compress(torch.randn(1, HKV, cached, D, device=dev, generator=g).to(torch.bfloat16))
    k1 = torch.randn(1, HKV, 1, D, device=dev, generator=g).to(torch.bfloat16)
    v1 = torch.randn(1, HKV, 1, D, device=dev, generator=g).to(torch.bfloat16)
    q1 = torch.randn(1, HQ, 1, D, device=dev, generator=g).to(torch.bfloat16)

    def step():
        kc.compress(k1)
        vc.compress(v1)
        return compressed_attention(q1, kc, vc, ck, cv, out_dtype=torch.bfloat16)

    for _ in range(20):
        step()
    torch.cuda.synchronize()
    e0, e1 = _events(2)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    host_us = (time.perf_counter() - t0) / steps * 1e6
    return {"workload": f"B1 Hq{HQ} Hkv{HKV} d{D} bits{BITS}, {cached} cached tokens, one new token per step",
            "host_us_per_step": host_us, "device_us_per_step": e0.elapsed_time(e1) / steps * 1e3}


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
        "workload": f"configs[1]: causal prefill B{B} Hq{HQ} Hkv{HKV} d{D} S{S} bits{BITS}: compress K/V + query prep + "
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
    ap.add_argument("--compress-only", action="store_true",
                    help="run only the north-star compression leg (1M key + 1M value rows) and print its record")
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

    if args.compress_only:
        print(json.dumps({"compress_north_star": compress_leg(kc, vc, args.steps, args.warmup)}), flush=True)
        return

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
        "config": {"workload": (f"north-star target: Llama-3-8B attention (Hq{HQ} Hkv{HKV} d{D} bits{BITS}) at "
                                f"{DEC_SK // 1024}k context, decode-shaped scoring: 1 query row x {DEC_B} sequences x "
                                f"{DEC_SK} keys per step, rotating over {DEC_ROT} caches"),
                   "global_batch": DEC_B, "seq_len": DEC_SK, "parallelism": "single-gpu",
                   "clock_settle_ms": SETTLE_MS},
        "roofline": scores_leg["roofline"],
        "compress_tokens_per_s": None if prefill is None else prefill["compress_tokens_per_s"],
        "decode_attention": attn_leg,
        "prefill": prefill,
        "decode_step": None if args.no_prefill else decode_step_leg(kc, vc),
        "compress_north_star": None if args.no_prefill else compress_leg(kc, vc, 5, 2),
    }
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline_decode(args.cpu_seconds / 2)
        if prefill is not None:
            prefill["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
