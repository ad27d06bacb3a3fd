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
row, MFMA roofline); one layer's eager decode step through the product path
(torch.ops.tq) at B = 1 with 4096 cached tokens, host and device time; the HBM
stream ceilings; compression at the north-star scale (1M key + 1M value rows);
the head_dim-64 (GPT-2) tiled path; and configs[2]'s 36-layer model forward
with its per-layer attention time.  CPU baselines: the build's torch CPU branch
of the reference's PyTorch path on bounded samples.  Prints one JSON line.  With --gpus N > 1 it exits: this build
runs on one GPU.
"""

from __future__ import annotations

import argparse
import ctypes
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
LEAD = 3  # untimed launches queued just before each decode leg's start event
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


class _TimedRanges:
    """Names the timed steps for a profiler: each timed loop runs inside a roctx range
    "timed:<leg>:<steps>" (roctxRangePushA / roctxRangePop).  A `rocprofv3 --kernel-trace
    --marker-trace` run of bench.py then records those ranges beside the kernels, and
    `bench.py --trace-summary` keeps, per range, the last <steps> dispatches of each kernel:
    the timed launches only, without the clock-settling, warm-up and lead-in launches that
    precede them.  Without the profiler the calls do nothing; without the roctx library they
    are skipped."""

    def __init__(self):
        self._lib = None
        for name in ("librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so"):
            try:
                self._lib = ctypes.CDLL(name)
                break
            except OSError:
                continue
        if self._lib is not None:
            self._lib.roctxRangePushA.argtypes = [ctypes.c_char_p]
        self._open = False

    def push(self, leg: str, steps: int):
        if self._lib is not None and not self._open:
            self._lib.roctxRangePushA(f"timed:{leg}:{steps}".encode())
            self._open = True

    def pop(self):
        if self._lib is not None and self._open:
            self._lib.roctxRangePop()
            self._open = False


RANGES = _TimedRanges()


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


def pmc_summary(paths: list[str], copy_mib: int) -> dict:
    """HBM traffic per dispatch from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE counter CSVs of a
    bench.py run with --calibrate-copy: per (kernel, grid size), the mean counter value (KiB) over
    its dispatches; the device-to-device copy of `copy_mib` MiB calibrates each counter (factor =
    true KiB / counted KiB), and traffic_bytes = (FETCH_SIZE * fetch_factor + WRITE_SIZE *
    write_factor) * 1024.  Each kernel's record is its dispatch group with the largest grid (the
    bench leg's workload)."""
    import csv

    def short(name: str) -> str:  # "void tq::k<2, 3>(tq::Args)" -> "tq::k<2, 3>"
        name = name[5:] if name.startswith("void ") else name
        return name[:name.rfind("(")] if name.endswith(")") and "(" in name else name

    sums: dict = {}
    for path in paths:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                key = (short(r["Kernel_Name"]), int(r["Grid_Size"]), r["Counter_Name"])
                acc = sums.setdefault(key, [0.0, 0])
                acc[0] += float(r["Counter_Value"])
                acc[1] += 1
    mean = {k: v[0] / v[1] for k, v in sums.items()}
    count = {k: v[1] for k, v in sums.items()}
    copy_kib = copy_mib * 1024.0
    copies = [k for k in mean if "copyBuffer" in k[0]]

    def biggest(name, counter):
        ks = [k for k in mean if k[0] == name and k[2] == counter]
        return max(ks, key=lambda k: k[1]) if ks else None

    cal = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        ks = [k for k in copies if k[2] == counter]
        k = max(ks, key=lambda k: mean[k]) if ks else None
        cal[counter] = copy_kib / mean[k] if k and mean[k] > 0 else None
    kernels = {}
    for name in sorted({k[0] for k in mean if "copyBuffer" not in k[0]}):
        kf, kw = biggest(name, "FETCH_SIZE"), biggest(name, "WRITE_SIZE")
        if kf is None or kw is None or None in cal.values():
            continue
        fetch, write = mean[kf], mean[kw]
        kernels[name] = {"grid_size": kf[1], "dispatches": count[kf], "fetch_kib": fetch, "write_kib": write,
                         "traffic_bytes": int(round((fetch * cal["FETCH_SIZE"] + write * cal["WRITE_SIZE"]) * 1024))}
    a, m = "tq::decode_attn_i8_kernel<2, 2, false, 1, 128>", "tq::decode_merge_kernel<128>"
    if a in kernels and m in kernels:
        kernels["decode_attention (attention + merge)"] = {
            "name": f"{a} + {m}", "traffic_bytes": kernels[a]["traffic_bytes"] + kernels[m]["traffic_bytes"]}
    return {"calibration": {"copy_bytes": copy_mib << 20, "fetch_factor": cal["FETCH_SIZE"],
                            "write_factor": cal["WRITE_SIZE"]},
            "sources": [os.path.basename(p) for p in paths],
            "method": ("mean counter KiB per dispatch per (kernel, grid size); the largest grid per kernel; "
                       "traffic_bytes = (FETCH_SIZE * fetch_factor + WRITE_SIZE * write_factor) * 1024"),
            "kernels": kernels}


def trace_summary(kernel_csv: str, marker_csv: str) -> str:
    """Markdown table of the timed launches in a `rocprofv3 --kernel-trace --marker-trace` run of
    bench.py: for every "timed:<leg>:<steps>" roctx range, the kernels that started and ended
    inside it, grouped by (kernel, grid size), each group cut to its last <steps> dispatches (the
    lead-in launches queued just before the range can still start inside it)."""
    import csv

    def short(name: str) -> str:
        name = name[5:] if name.startswith("void ") else name
        return name[:name.rfind("(")] if name.endswith(")") and "(" in name else name

    ranges = []
    with open(marker_csv, newline="") as f:
        for r in csv.DictReader(f):
            msg = next((r[c] for c in ("Function", "Message", "Name", "Operation") if r.get(c, "").startswith("timed:")),
                       None)
            if msg is None:
                continue
            _, leg, steps = msg.split(":")
            ranges.append((leg, int(steps), int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    kernels = []
    with open(kernel_csv, newline="") as f:
        for r in csv.DictReader(f):
            grid = int(r["Grid_Size"]) if "Grid_Size" in r else (
                int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"]))
            kernels.append((short(r["Kernel_Name"]), grid, int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    kernels.sort(key=lambda k: k[2])
    lines = ["| timed range (steps) | kernel | grid (work-items) | launches per step | avg us | min us | max us | "
             "us per step |", "|---|---|---|---|---|---|---|---|"]
    for leg, steps, t0, t1 in sorted(ranges, key=lambda r: r[2]):
        groups: dict = {}
        for name, grid, k0, k1 in kernels:
            if t0 <= k0 and k1 <= t1:
                groups.setdefault((name, grid), []).append((k1 - k0) / 1e3)
        rows = []
        for (name, grid), us in groups.items():
            per_step = max(1, round(len(us) / steps))  # lead-in launches aside
            last = us[-steps * per_step:]
            avg = sum(last) / len(last)
            rows.append((avg * per_step, name, grid, per_step, avg, min(last), max(last)))
        for tot, name, grid, per_step, avg, lo, hi in sorted(rows, reverse=True)[:12]:
            short = name if len(name) <= 72 else name[:69] + "..."
            lines.append(f"| {leg} ({steps}) | `{short}` | {grid} | {per_step} | {avg:.1f} | {lo:.1f} | {hi:.1f} | "
                         f"{tot:.1f} |")
    return "\n".join(lines)


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
    # fresh queries per step for the API-level step (query preparation + scores)
    qs = [torch.randn(DEC_B, HQ, 1, D, device=dev, generator=gen).to(torch.bfloat16) for _ in range(DEC_ROT)]
    q = qs[0]
    q_rot, q_proj = kc.prepare_queries(q)
    api_rot = [torch.empty_like(q_rot) for _ in range(DEC_ROT)]
    api_proj = [torch.empty_like(q_proj) for _ in range(DEC_ROT)]
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

    def launch_api(i):
        # the reference's scoring call (compressors.py:178-200 with attention.py:158-167): rotate and
        # project this step's queries, then score them against the compressed keys
        j = i % DEC_ROT
        qj, ck = qs[j], caches[j][0]
        st = lib.tq_query_prep(qj.data_ptr(), _native.TQ_BF16, DEC_B, HQ, 1, D, qj.stride(0), qj.stride(1),
                               qj.stride(2), tk.pi_split.data_ptr(), tk.s_eff16.data_ptr(), api_rot[j].data_ptr(),
                               api_proj[j].data_ptr(), stream)
        if st:
            return st
        return lib.tq_attention_scores(
            api_rot[j].data_ptr(), api_proj[j].data_ptr(), ck["packed_key_indices"].data_ptr(),
            ck["packed_qjl_signs"].data_ptr(), ck["residual_norm"].data_ptr(), ck["vec_norms"].data_ptr(),
            tk.cent16.data_ptr(), DEC_B, HQ, HKV, 1, DEC_SK, D, BITS, coeff, scores[j].data_ptr(), stream)

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

    def timed(launch, leg):
        settle_clock(launch)
        for i in range(warmup):
            _native.check(launch(i), "decode warmup")
        torch.cuda.synchronize()
        # a few untimed launches queued right before the start event keep the stream busy while
        # the host issues the first timed one: the events then hold the K timed steps back to
        # back, not the host's latency to its first launch after an idle GPU
        for i in range(LEAD):
            _native.check(launch(i), "decode lead-in")
        RANGES.push(leg, steps)
        e0, e1 = _events(2)
        e0.record()
        for i in range(steps):
            st = launch(i)
            if st:
                _native.check(st, "decode launch")
        e1.record()
        torch.cuda.synchronize()
        RANGES.pop()
        return e0.elapsed_time(e1) / steps

    ms_scores = timed(launch_scores, "decode_scores")
    ms_api = timed(launch_api, "api_step")
    ms_attn = timed(launch_attn, "decode_attention")
    key_heads = DEC_B * HQ * DEC_SK
    q_bytes = DEC_B * HQ * D * (2 + 4)  # prepared queries read: f16 q_rot + f32 q_proj
    score_bytes = DEC_B * HKV * DEC_SK * key_rec_bytes(BITS, D) + key_heads * 4 + q_bytes
    # the API step also reads the bf16 queries and writes the prepared ones
    api_bytes = score_bytes + DEC_B * HQ * D * (2 + 2 + 4)
    attn_bytes = (DEC_B * HKV * DEC_SK * (key_rec_bytes(BITS, D) + val_rec_bytes(BITS, D)) + q_bytes
                  + DEC_B * HQ * D * 2)
    gbs_s = score_bytes / (ms_scores * 1e-3) / 1e9
    gbs_api = api_bytes / (ms_api * 1e-3) / 1e9
    gbs_a = attn_bytes / (ms_attn * 1e-3) / 1e9
    scores_leg = {
        "ms_per_launch": ms_scores,
        "key_heads_per_s": key_heads / (ms_scores * 1e-3),
        "roofline": {
            "kernel": "tq::decode_scores_i8_kernel<2, 3, 1, 128> (scores, f32 written)",
            "bound": "hbm", "achieved": gbs_s, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": gbs_s / HBM_PEAK_GBS, "traffic": measured_traffic("tq::decode_scores_i8_kernel<2, 3, 1, 128>"),
            "algorithmic_bytes_per_launch": score_bytes,
        },
        "api_step": {
            "what": ("the reference's scoring call per step: tq_query_prep (rotate + project this step's "
                     f"{DEC_B}x{HQ} bf16 query rows) then tq_attention_scores, fresh queries every step"),
            "ms_per_step": ms_api,
            "key_heads_per_s": key_heads / (ms_api * 1e-3),
            "roofline": {"bound": "hbm", "achieved": gbs_api, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": gbs_api / HBM_PEAK_GBS, "algorithmic_bytes_per_step": api_bytes},
        },
    }
    attn_leg = {
        "workload": f"fused decode attention, same caches: B{DEC_B} Hq{HQ} Hkv{HKV} Sq1 Sk{DEC_SK} bits{BITS}",
        "ms_per_launch": ms_attn,
        "key_heads_per_s": key_heads / (ms_attn * 1e-3),
        "roofline": {
            "kernel": "tq::decode_attn_i8_kernel<2, 2, false, 1, 128> + tq::decode_merge_kernel<128>",
            "bound": "hbm", "achieved": gbs_a, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": gbs_a / HBM_PEAK_GBS, "traffic": measured_traffic("decode_attention (attention + merge)"),
            "algorithmic_bytes_per_launch": attn_bytes,
        },
    }
    del caches, scores, outs, ws, api_rot, api_proj
    torch.cuda.empty_cache()
    return scores_leg, attn_leg


def hbm_ceiling_leg(steps: int, warmup: int) -> dict:
    """What the memory system delivers to a kernel that only streams, measured in the same run as
    the headline (csrc/tq_probe.hip: non-temporal 16-byte loads and stores, as the decode kernels
    issue them): read-only over the headline's 218 MB of key planes, write-only over its 67 MB of
    scores, and the two mixed 13 KiB : 4 KiB per wave as the scores kernel mixes them; each over
    DEC_ROT rotating buffers, the best of three grid sizes."""
    import torch

    from turboquant_pytorch import _native

    path = os.path.join(os.path.dirname(_native.library_path()), "libtq_probe.so")
    probe = ctypes.CDLL(path)
    probe.tq_probe_stream.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                      ctypes.c_int32, ctypes.c_void_p]
    probe.tq_probe_unit_bytes.restype = ctypes.c_int64
    probe.tq_probe_unit_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32]
    read_total = DEC_B * HKV * DEC_SK * key_rec_bytes(BITS, D)
    write_total = DEC_B * HQ * DEC_SK * 4
    stream = torch.cuda.current_stream().cuda_stream
    out = {}
    for name, mode, units in (("read_only", 0, read_total // probe.tq_probe_unit_bytes(0, 0)),
                              ("write_only", 1, write_total // probe.tq_probe_unit_bytes(1, 1)),
                              ("mix_13_4", 2, read_total // probe.tq_probe_unit_bytes(2, 0))):
        rb, wb = units * probe.tq_probe_unit_bytes(mode, 0), units * probe.tq_probe_unit_bytes(mode, 1)
        srcs = [torch.empty(max(rb, 16), dtype=torch.uint8, device="cuda").fill_(i + 1) for i in range(DEC_ROT)]
        dsts = [torch.empty(max(wb, 4096), dtype=torch.uint8, device="cuda") for _ in range(DEC_ROT)]
        best = None
        for blocks in (1024, 2048, 4096):
            def launch(i):
                return probe.tq_probe_stream(srcs[i % DEC_ROT].data_ptr(), dsts[i % DEC_ROT].data_ptr(), units,
                                             mode, blocks, stream)
            settle_clock(launch, SETTLE_MS / 4)
            for i in range(warmup):
                _native.check(launch(i), "probe warmup")
            torch.cuda.synchronize()
            for i in range(LEAD):
                _native.check(launch(i), "probe lead-in")
            e0, e1 = _events(2)
            e0.record()
            for i in range(steps):
                _native.check(launch(i), "probe")
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / steps * 1e3
            if best is None or us < best[0]:
                best = (us, blocks)
        us, blocks = best
        gbs = (rb + wb) / (us * 1e-6) / 1e9
        out[name] = {"read_bytes": rb, "write_bytes": wb, "us_per_launch": us, "gbs": gbs,
                     "frac_of_peak": gbs / HBM_PEAK_GBS, "blocks": blocks}
        del srcs, dsts
    torch.cuda.empty_cache()
    return out


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
        for _ in range(2):  # lead-in: the stream is busy when the start event is recorded
            fn(x)
        RANGES.push(f"compress_{name}", steps)
        e0, e1 = _events(2)
        e0.record()
        for _ in range(steps):
            fn(x)
        e1.record()
        torch.cuda.synchronize()
        RANGES.pop()
        us = e0.elapsed_time(e1) / steps * 1e3
        gbs = rows * (2 * D + rec) / (us * 1e-6) / 1e9
        tflops = rows * passes * 2 * D * D / (us * 1e-6) / 1e12
        out[name] = {"us_per_launch": us, "rows_per_s": rows / (us * 1e-6), "hbm_gbs": gbs,
                     "hbm_frac": gbs / HBM_PEAK_GBS, "mfma_tflops": tflops,
                     "mfma_frac": tflops / MFMA_F16_PEAK_TFLOPS}
    both = out["keys"]["us_per_launch"] + out["values"]["us_per_launch"]
    return {"workload": f"B4 Hkv{HKV} S32768 d{D} bf16 bits{BITS}: {rows} key rows + {rows} value rows",
            "tokens_per_s": 4 * 32768 / (both * 1e-6), **out}


def decode_step_leg(kc, vc, steps: int = 200, hq: int = HQ, hkv: int = HKV, d: int = D,
                    shapes=((1, 4096), (1, 32768), (16, 4096), (16, 32768)), label: str = "decode_step") -> dict:
    """One attention layer's decode step on the cached serving path (TurboQuantCache, as a patched
    layer runs it under generate, TurboQuantCache.append_attend: one tq::cache_attend operator call):
    tq::cache_append compresses the new token's K and V (hkv kv heads, 8 by default) straight into
    the cache planes and prepares the hq query heads' query (32) in one launch, then the split-K
    attention over every cached position (attention + merge).  bits 3, B
    and cached tokens from `shapes` (1 and 16 x 4096 and 32768 by default); the cache is sized
    beforehand so that no step grows it.  Host time
    per step (wall clock over `steps` back-to-back steps, synchronised at the end) and device time
    (HIP events around the same steps)."""
    import torch

    from transformers_turboquant import TurboQuantCache

    dev = "cuda"
    out = {}
    warm = 20
    for b_, cached in shapes:
        g = torch.Generator(device=dev).manual_seed(5 + b_ + cached)
        cache = TurboQuantCache()
        total = cached + warm + steps
        for lo in range(0, total, 8192):  # prefill in chunks; then keep `cached` positions
            n = min(8192, total - lo)
            cache.append(0, kc, vc, torch.randn(b_, hkv, n, d, device=dev, generator=g).to(torch.bfloat16),
                         torch.randn(b_, hkv, n, d, device=dev, generator=g).to(torch.bfloat16))
        cache.layer(0).crop(cached)
        k1 = torch.randn(b_, hkv, 1, d, device=dev, generator=g).to(torch.bfloat16)
        v1 = torch.randn(b_, hkv, 1, d, device=dev, generator=g).to(torch.bfloat16)
        q1 = torch.randn(b_, hq, 1, d, device=dev, generator=g).to(torch.bfloat16)

        def step():
            return cache.append_attend(0, kc, vc, k1, v1, q1, out_dtype=torch.bfloat16)

        for _ in range(warm):
            step()
        cache.layer(0).crop(cached)
        torch.cuda.synchronize()
        RANGES.push(f"{label}_B{b_}_S{cached}", steps)
        e0, e1 = _events(2)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            step()
        e1.record()
        torch.cuda.synchronize()
        host_us = (time.perf_counter() - t0) / steps * 1e6
        RANGES.pop()
        out[f"B{b_}_S{cached}"] = {"host_us_per_step": host_us, "device_us_per_step": e0.elapsed_time(e1) / steps * 1e3}
        del cache
        torch.cuda.empty_cache()
    return {"workload": (f"Hq{hq} Hkv{hkv} d{d} bits{BITS}: one new token per step appended to a TurboQuantCache "
                         "(one launch: K, V and query preparation) + split-K attention over every cached position"),
            **out}


def head_dim64_leg(steps: int, warmup: int) -> dict:
    """The head_dim-64 path (GPT-2's attention, BASELINE.json configs[0]'s shape: 12 heads, bits 3)
    through the prefill kernel at head_dim 64: one layer's compress K / V + query prep + fused attention per step,
    at configs[0]'s 512 tokens and at 8192 tokens (causal), HIP events around the attention call
    and around the whole step; and one decode step's attention (one query row over 4k / 32k
    cached keys) through the split-K decode kernel at head_dim 64."""
    import torch

    from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2
    from turboquant_pytorch.fused import attention_from_prepared

    d, h = 64, 12
    kc = TurboQuantCompressorV2(d, BITS, seed=42, device="cuda")
    vc = TurboQuantCompressorMSE(d, BITS, seed=10042, device="cuda")
    out = {}
    for S_ in (512, 8192):
        g = torch.Generator(device="cuda").manual_seed(S_)
        q, k, v = (torch.randn(1, h, S_, d, device="cuda", generator=g).to(torch.bfloat16) for _ in range(3))
        marks = []

        def step(record):
            e = _events(3) if record else None
            if record:
                e[0].record()
            ck, cv = kc.compress(k), vc.compress(v)
            q_rot, q_proj = kc.prepare_queries(q)
            if record:
                e[1].record()
            attention_from_prepared(q_rot, q_proj, kc, vc, ck, cv, causal=True, out_dtype=torch.bfloat16)
            if record:
                e[2].record()
                marks.append(e)

        for _ in range(warmup + 1):
            step(False)
        torch.cuda.synchronize()
        RANGES.push(f"head_dim64_S{S_}", steps)
        for _ in range(steps):
            step(True)
        torch.cuda.synchronize()
        RANGES.pop()
        attn_ms = sorted(m[1].elapsed_time(m[2]) for m in marks)[len(marks) // 2]
        step_ms = sorted(m[0].elapsed_time(m[2]) for m in marks)[len(marks) // 2]
        key_heads = h * S_ * (S_ + 1) // 2
        tflops = key_heads * 6 * d / (attn_ms * 1e-3) / 1e12
        out[f"S{S_}"] = {"step_ms": step_ms, "attention_ms": attn_ms, "attention_tflops": tflops,
                         "mfma_frac": tflops / MFMA_F16_PEAK_TFLOPS}
    # one decode step's attention over a compressed cache at this head dim (one query row per
    # sequence): the split-K decode kernel (bit planes) + merge
    for b_, sk in ((1, 4096), (1, 32768)):
        g = torch.Generator(device="cuda").manual_seed(sk)
        ck = kc.compress(torch.randn(b_, h, sk, d, device="cuda", generator=g).to(torch.bfloat16))
        cv = vc.compress(torch.randn(b_, h, sk, d, device="cuda", generator=g).to(torch.bfloat16))
        q_rot, q_proj = kc.prepare_queries(torch.randn(b_, h, 1, d, device="cuda", generator=g).to(torch.bfloat16))
        for _ in range(warmup + 5):
            attention_from_prepared(q_rot, q_proj, kc, vc, ck, cv, out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        RANGES.push(f"head_dim64_decode_B{b_}_S{sk}", steps)
        e0, e1 = _events(2)
        e0.record()
        for _ in range(steps):
            attention_from_prepared(q_rot, q_proj, kc, vc, ck, cv, out_dtype=torch.bfloat16)
        e1.record()
        torch.cuda.synchronize()
        RANGES.pop()
        out[f"decode_B{b_}_S{sk}"] = {"attention_us": e0.elapsed_time(e1) / steps * 1e3}
    # the cached serving step at this shape (append + attention over every cached position)
    out["decode_step"] = decode_step_leg(kc, vc, steps=max(steps, 50), hq=h, hkv=h, d=d,
                                         shapes=((1, 4096), (1, 32768)), label="head_dim64_decode_step")
    return {"workload": f"GPT-2 attention shape: B1 x {h} heads x d{d}, bits {BITS}, causal; "
                        "tq::prefill_kernel<64, 3, false> (q_proj as f16 hi + lo); decode steps (one query "
                        "row over 4k / 32k cached keys) through tq::decode_attn_i8_kernel<2, 3, false, 1, 64> "
                        "+ merge",
            **out}


def model_leg(steps: int = 3, S_model: int = 8192, bits: int = BITS) -> dict:
    """the 36-layer Qwen2.5-3B-shaped random-init model (hidden 2048, 16 / 2
    heads, head_dim 128, bf16) patched by apply_turboquant (bits 3, seed 42, the reference's
    defaults), one full-sequence forward of 8192 uniform-random token ids with logits_to_keep=1.
    Whole-forward time (HIP events around each forward) and the time of every patched attention
    module (events in forward pre / post hooks: q/k/v projections, rotary, K / V compression,
    query preparation, fused attention, o_proj), summed over the layers."""
    import torch
    from transformers import Qwen2Config, Qwen2ForCausalLM

    from transformers_turboquant import apply_turboquant

    cfg = Qwen2Config(vocab_size=151936, hidden_size=2048, intermediate_size=11008, num_hidden_layers=36,
                      num_attention_heads=16, num_key_value_heads=2, max_position_embeddings=32768,
                      tie_word_embeddings=True)
    torch.manual_seed(0)
    with torch.device("cuda"):
        model = Qwen2ForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    apply_turboquant(model, bits=bits, seed=42)
    ids = torch.randint(0, cfg.vocab_size, (1, S_model), generator=torch.Generator().manual_seed(0)).to("cuda")
    marks = []

    record = [False]

    def pre(mod, args, kwargs):
        if record[0]:
            e = _events(2)
            e[0].record()
            marks.append(e)

    def post(mod, args, kwargs, out):
        if record[0]:
            marks[-1][1].record()

    handles = []
    for layer in model.model.layers:
        handles.append(layer.self_attn.register_forward_pre_hook(pre, with_kwargs=True))
        handles.append(layer.self_attn.register_forward_hook(post, with_kwargs=True))
    with torch.no_grad():
        model(input_ids=ids, logits_to_keep=1)
        torch.cuda.synchronize()
        record[0] = True
        fwd = []
        RANGES.push("model_forward", steps)
        for _ in range(steps):
            e = _events(2)
            e[0].record()
            model(input_ids=ids, logits_to_keep=1)
            e[1].record()
            fwd.append(e)
        torch.cuda.synchronize()
        RANGES.pop()
    for h in handles:
        h.remove()
    fwd_ms = sorted(e[0].elapsed_time(e[1]) for e in fwd)[len(fwd) // 2]
    n_layers = cfg.num_hidden_layers
    attn_ms = sum(m[0].elapsed_time(m[1]) for m in marks) / steps
    del model
    torch.cuda.empty_cache()
    return {"workload": (f"configs[2]: Qwen2.5-3B-shaped random-init model, 36 layers, bf16, B1 x {S_model} tokens, "
                         f"bits {bits}, apply_turboquant defaults (non-causal as the reference), logits_to_keep=1"),
            "forward_ms": fwd_ms, "tokens_per_s": S_model / (fwd_ms * 1e-3),
            "attention_modules_ms": attn_ms, "attention_ms_per_layer": attn_ms / n_layers,
            "attention_share": attn_ms / fwd_ms}


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
    step(False)  # lead-in: the stream is busy when the first timed step's events are recorded
    RANGES.push("prefill", steps)
    t0 = time.perf_counter()
    for _ in range(steps):
        step(True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    RANGES.pop()
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
            "kernel": "tq::prefill_kernel<128, 3, false> (fused scores + softmax + P.V; q_proj as f16 hi + lo)",
            "bound": "mfma", "achieved": tflops, "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / MFMA_F16_PEAK_TFLOPS, "traffic": measured_traffic("tq::prefill_kernel<128, 3, false>"),
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
    ap.add_argument("--no-ceiling", action="store_true", help="skip the HBM stream-ceiling leg")
    ap.add_argument("--no-model", action="store_true", help="skip the whole-model forward leg")
    ap.add_argument("--compress-only", action="store_true",
                    help="run only the north-star compression leg (1M key + 1M value rows) and print its record")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="run one device-to-device copy of MIB MiB first (PMC byte-counter calibration)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="CSV",
                    help="summarise rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE counter CSVs of a bench run "
                         "(with --calibrate-copy) into the traffic record; no GPU work")
    ap.add_argument("--copy-mib", type=int, default=256, help="size of the calibration copy in those CSVs")
    ap.add_argument("--trace-summary", nargs=2, metavar=("KERNEL_CSV", "MARKER_CSV"),
                    help="summarise the timed launches of a rocprofv3 --kernel-trace --marker-trace run of "
                         "bench.py (kernel_trace.csv, marker_api_trace.csv); no GPU work")
    args = ap.parse_args()
    if args.trace_summary:
        print(trace_summary(*args.trace_summary))
        return
    if args.pmc_summary:
        print(json.dumps(pmc_summary(args.pmc_summary, args.copy_mib), indent=1))
        return
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
    ceiling = None if args.no_ceiling else hbm_ceiling_leg(args.steps, args.warmup)
    if ceiling is not None:
        mix = ceiling["mix_13_4"]["gbs"]
        ceiling["scores_kernel_of_mix"] = scores_leg["roofline"]["achieved"] / mix
        ceiling["api_step_of_mix"] = scores_leg["api_step"]["roofline"]["achieved"] / mix
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
        "dtype": ("int8-mfma bit-plane keys x 24-bit fixed-point queries (four int8 digits, exact int32 sums: "
                  "f32-grade q_rot.C and q_proj), f32 scores"),
        "data": "synthetic (bf16 N(0,1) Q/K/V, 4 K channels x20 = randperm(128, seed 1)[:4]; seeds 0 and 2)",
        "config": {"workload": (f"north-star target: Llama-3-8B attention (Hq{HQ} Hkv{HKV} d{D} bits{BITS}) at "
                                f"{DEC_SK // 1024}k context, decode-shaped scoring: 1 query row x {DEC_B} sequences x "
                                f"{DEC_SK} keys per step, rotating over {DEC_ROT} caches"),
                   "global_batch": DEC_B, "seq_len": DEC_SK, "parallelism": "single-gpu",
                   "clock_settle_ms": SETTLE_MS},
        "roofline": scores_leg["roofline"],
        "api_step": scores_leg["api_step"],
        "hbm_ceiling": ceiling,
        "compress_tokens_per_s": None if prefill is None else prefill["compress_tokens_per_s"],
        "decode_attention": attn_leg,
        "prefill": prefill,
        "decode_step": None if args.no_prefill else decode_step_leg(kc, vc),
        "compress_north_star": None if args.no_prefill else compress_leg(kc, vc, 5, 2),
        "head_dim64": None if args.no_prefill else head_dim64_leg(args.steps, args.warmup),
        "model_forward": None if (args.no_prefill or args.no_model) else model_leg(),
    }
    if not args.no_cpu_baseline:
        rec["cpu_baseline"] = cpu_baseline_decode(args.cpu_seconds / 2)
        if prefill is not None:
            prefill["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
