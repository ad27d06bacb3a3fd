"""Validation metrics for TurboQuant key compression (reference: validate.py, tests/test_slow.py).

The reference's harness captures a model's per-layer K/V after one forward pass,
compresses each layer's keys with ``TurboQuantCompressorV2(d, bits,
seed=layer*1000)`` and its values with ``TurboQuantCompressorMSE(d, bits,
seed=layer*1000+500)`` (validate.py:120-132), takes the last key of each head
as a proxy query (:163), and compares the exact scores ``q.k`` with the
compressed-domain estimate per head: cosine similarity of the score vectors,
top-1 agreement, whether the exact top-1 key is in the estimate's top 5, and
the rank of a "needle" position in the estimate (:168-199).  Storage is counted
per bit (:137-152).  test_slow.py:79-93 adds the variance of the scores over
keys.

Here every metric is computed for all heads at once on the scores' device (no
per-head host round trips), the scores come from the packed GPU path when the
cache lives on the GPU, and the cache can come from a local model checkpoint or
from ``synthetic_needle_cache`` (no network is needed).  Differences from the
reference reporter, on purpose: a needle at position 0 is reported (the
reference's ``if needle_start`` drops it), and ties in the needle's rank are
broken by position (the reference's unstable ``argsort`` leaves them open).
"""

from __future__ import annotations

import argparse
import json
import time
from dataclasses import asdict, dataclass, field

import torch
import torch.nn.functional as F

from .compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

__all__ = [
    "storage_bits", "packed_nbytes", "score_metrics", "score_variance", "find_subsequence",
    "build_prompt", "synthetic_needle_cache", "capture_cache", "validate_cache", "BitsReport", "main",
]

KEY_SEED_STRIDE = 1000   # validate.py:127
VALUE_SEED_OFFSET = 500  # validate.py:130


def storage_bits(n_vecs: int, d: int, bits: int) -> tuple[int, int]:
    """(key bits, value bits) TurboQuant stores for n_vecs key and value vectors (validate.py:137-152).

    Keys: (bits-1)-bit codes (at least 1), one QJL sign bit per coordinate, f16
    residual and vector norms.  Values: bits-bit codes and an f16 vector norm.
    """
    mse_bits = max(bits - 1, 1)
    k = n_vecs * (d * mse_bits + d + 16 + 16)
    v = n_vecs * (d * bits + 16)
    return k, v


def packed_nbytes(compressed: dict) -> int:
    """Bytes the tensors of a compressed dict occupy (its actual storage, row padding included)."""
    return sum(t.numel() * t.element_size() for t in compressed.values() if isinstance(t, torch.Tensor))


@dataclass
class HeadMetrics:
    cosine: torch.Tensor       # f32 [N]
    top1: torch.Tensor         # bool [N]
    top5: torch.Tensor         # bool [N]
    needle_rank: torch.Tensor | None  # int64 [N]


def score_metrics(real: torch.Tensor, est: torch.Tensor, needle: int | None = None) -> HeadMetrics:
    """Per score vector (last dim = keys) metrics of validate.py:168-199, for all rows at once.

    cosine: ``F.cosine_similarity`` of the two vectors (:171); top1: the argmax
    positions agree (:175-178); top5: the exact argmax is among the estimate's 5
    largest (:181-183); needle_rank: 0-based position of key `needle` when the
    estimate is sorted in descending order (:186-191).  Ties in the estimate are
    broken by position for both (the reference's topk/argsort leave them open).
    """
    if real.shape != est.shape:
        raise ValueError(f"score shapes differ: {tuple(real.shape)} vs {tuple(est.shape)}")
    S = real.shape[-1]
    r = real.reshape(-1, S).float()
    e = est.reshape(-1, S).float().to(r.device)
    cos = F.cosine_similarity(r, e, dim=-1)
    r1 = r.argmax(dim=-1)
    top1 = e.argmax(dim=-1) == r1
    top5 = _stable_rank(e, r1[:, None]) < 5
    rank = None
    if needle is not None:
        if not 0 <= needle < S:
            raise ValueError(f"needle position {needle} outside [0, {S})")
        rank = _stable_rank(e, torch.full((e.shape[0], 1), needle, device=e.device))
    return HeadMetrics(cos, top1, top5, rank)


def _stable_rank(e: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
    """0-based place of column pos[i] in row i of e sorted descending, ties by position."""
    v = e.gather(1, pos)
    before = torch.arange(e.shape[1], device=e.device)[None, :] < pos
    return (e > v).sum(dim=-1) + ((e == v) & before).sum(dim=-1)


def score_variance(scores: torch.Tensor) -> torch.Tensor:
    """Variance of [B, H, S_q, S_k] scores over keys, averaged over batch and query rows: [H] (test_slow.py:79-93)."""
    return scores.float().var(dim=-1).mean(dim=(0, 2))


def find_subsequence(ids: list[int], pattern: list[int]) -> int | None:
    """First position of `pattern` in `ids`; failing that, of its longest prefix found (validate.py:80-97)."""
    for width in range(len(pattern), 0, -1):
        sub = pattern[:width]
        for i in range(len(ids) - width + 1):
            if ids[i:i + width] == sub:
                return i
    return None


# A haystack of unrelated prose with one planted fact, asked about at the end.
HAYSTACK = (
    "The river authority published its annual survey of the northern basin. Water levels\n"
    "stayed within seasonal norms, two pumping stations were refitted, and the volunteer\n"
    "program counted more wading birds than in any year since records began. The report\n"
    "closes with a schedule of public meetings and a list of culverts due for inspection.\n\n"
)
NEEDLE = "The vault access phrase is COBALT-3162."
QUESTION = "What is the vault access phrase?"
NEEDLE_KEY = "COBALT-3162"


def build_prompt(tokenizer, target_tokens: int = 2048, needle_pos: float = 0.5, haystack: str = HAYSTACK,
                 needle: str = NEEDLE, question: str = QUESTION) -> str:
    """Repeat `haystack` to about `target_tokens` tokens with `needle` planted at fraction
    `needle_pos`, then ask `question` (the construction of validate.py:32-45).  The text
    is wrapped in the tokenizer's chat template when it has one."""
    unit = len(tokenizer.encode(haystack))
    reps = max(1, target_tokens // max(unit, 1))
    at = int(reps * needle_pos)
    parts = []
    for i in range(reps):
        if i == at:
            parts.append(f"\n--- Memo ---\n{needle}\n--- End ---\n\n")
        parts.append(haystack)
    user = "".join(parts) + f"\nQuestion: {question}"
    if getattr(tokenizer, "chat_template", None):
        return tokenizer.apply_chat_template([{"role": "user", "content": user}], tokenize=False,
                                             add_generation_prompt=True)
    return user


def synthetic_needle_cache(n_layers: int = 4, batch: int = 1, heads: int = 8, seq: int = 2048, head_dim: int = 128,
                           needle_pos: float = 0.5, outlier_channels: int = 4, outlier_bias: float = 4.0,
                           needle_gain: float = 0.6, noise: float = 0.3, seed: int = 0, device="cpu",
                           dtype=torch.bfloat16) -> tuple[list[tuple[torch.Tensor, torch.Tensor]], int]:
    """Per-layer (keys, values) [B, H, S, D] with LLM-like key statistics and a planted needle.

    Keys are N(0, 1) plus a constant offset of +-outlier_bias on a few channels
    (the channel-wise bias real attention keys carry).  The last key, the
    harness's proxy query, is needle_gain * (needle key) + noise * N(0, 1), with
    the channel offset restored; at the defaults the needle is the exact top-1
    key of (nearly) every head, ahead of the query's own position.  Returns
    (layers, needle position).
    """
    g = torch.Generator().manual_seed(seed)
    needle = int((seq - 1) * needle_pos)
    chans = torch.randperm(head_dim, generator=g)[:outlier_channels]
    offset = outlier_bias * (torch.randint(0, 2, (outlier_channels,), generator=g) * 2.0 - 1.0)
    layers = []
    for _ in range(n_layers):
        k = torch.randn(batch, heads, seq, head_dim, generator=g)
        k[..., chans] += offset
        k[:, :, -1] = needle_gain * k[:, :, needle] + noise * torch.randn(batch, heads, head_dim, generator=g)
        k[:, :, -1, chans] += (1.0 - needle_gain) * offset
        v = torch.randn(batch, heads, seq, head_dim, generator=g)
        layers.append((k.to(device, dtype), v.to(device, dtype)))
    return layers, needle


def capture_cache(model, input_ids: torch.Tensor, attention_mask: torch.Tensor | None = None):
    """One forward pass with the model's own cache; returns per-layer (keys, values) (validate.py:101-107)."""
    with torch.no_grad():
        out = model(input_ids=input_ids, attention_mask=attention_mask, use_cache=True)
    cache = out.past_key_values
    return [(lay.keys, lay.values) for lay in cache.layers]


@dataclass
class BitsReport:
    bits: int
    n_checks: int
    compressed_bytes: float        # per-bit accounting (validate.py:137-152)
    uncompressed_bytes: int        # f16 K and V
    ratio: float
    packed_bytes: int              # actual bytes of the compressed dicts
    cosine: float
    top1_pct: float
    top5_pct: float
    needle_rank: float             # mean over heads; -1 without a needle
    seconds: float
    variance: dict = field(default_factory=dict)   # layer -> per-head |estimate - exact| score variance


@torch.no_grad()
def validate_cache(layers, bits_list=(2, 3, 4), needle: int | None = None,
                   with_variance: bool = False) -> list[BitsReport]:
    """The reference's per-bit report (validate.py:115-225) over captured or synthetic layers.

    layers: sequence of (keys, values) [B, H, S, D]; the query is the last key
    of each head.  Scores use the compressed dicts in the format the cache's
    device produces (packed on the GPU, unpacked on the CPU).
    """
    reports = []
    for bits in bits_list:
        t0 = time.perf_counter()
        comp_bits = 0
        raw_bytes = 0
        packed = 0
        cos, top1, top5, ranks = [], [], [], []
        var = {}
        for li, (keys, values) in enumerate(layers):
            B, H, S, D = keys.shape
            dev = str(keys.device)
            kc = TurboQuantCompressorV2(D, bits, seed=li * KEY_SEED_STRIDE, device=dev)
            vc = TurboQuantCompressorMSE(D, bits, seed=li * KEY_SEED_STRIDE + VALUE_SEED_OFFSET, device=dev)
            ck = kc.compress(keys)
            cv = vc.compress(values)
            packed += packed_nbytes(ck) + packed_nbytes(cv)
            kb, vb = storage_bits(B * H * S, D, bits)
            comp_bits += kb + vb
            raw_bytes += (keys.numel() + values.numel()) * 2
            q = keys[:, :, -1:, :]
            real = torch.matmul(q.float(), keys.float().transpose(-2, -1))
            est = kc.asymmetric_attention_scores(q, ck)
            m = score_metrics(real, est, needle)
            cos.append(m.cosine)
            top1.append(m.top1)
            top5.append(m.top5)
            if m.needle_rank is not None:
                ranks.append(m.needle_rank)
            if with_variance:
                var[li] = (score_variance(est) - score_variance(real)).abs().tolist()
        cos_all = torch.cat(cos)
        n = cos_all.numel()
        if torch.cuda.is_available():
            torch.cuda.synchronize()
        comp_bytes = comp_bits / 8
        reports.append(BitsReport(
            bits=bits, n_checks=n, compressed_bytes=comp_bytes, uncompressed_bytes=raw_bytes,
            ratio=raw_bytes / comp_bytes, packed_bytes=packed, cosine=float(cos_all.double().mean()),
            top1_pct=100.0 * float(torch.cat(top1).double().mean()),
            top5_pct=100.0 * float(torch.cat(top5).double().mean()),
            needle_rank=float(torch.cat(ranks).double().mean()) if ranks else -1.0,
            seconds=time.perf_counter() - t0, variance=var))
    return reports


def format_report(rep: BitsReport) -> str:
    mb = 1024 * 1024
    lines = [
        f"  TQ-{rep.bits}bit:",
        f"    Compression:       {rep.ratio:.1f}x  ({rep.compressed_bytes / mb:.1f} MB vs "
        f"{rep.uncompressed_bytes / mb:.1f} MB; stored dicts {rep.packed_bytes / mb:.1f} MB)",
        f"    Score cosine sim:  {rep.cosine:.6f}",
        f"    Top-1 match:       {rep.top1_pct:.1f}%  ({round(rep.top1_pct * rep.n_checks / 100)}/{rep.n_checks} heads)",
        f"    Top-5 match:       {rep.top5_pct:.1f}%",
    ]
    if rep.needle_rank >= 0:
        lines.append(f"    Avg needle rank:   {rep.needle_rank:.1f}  (0 = top)")
    return "\n".join(lines)


def _model_cases(path: str, tokens: list[int], device: str):
    from transformers import AutoModelForCausalLM, AutoTokenizer

    tok = AutoTokenizer.from_pretrained(path, local_files_only=True)
    model = AutoModelForCausalLM.from_pretrained(path, local_files_only=True, dtype=torch.float16).to(device).eval()
    pattern = tok.encode(NEEDLE_KEY, add_special_tokens=False)
    for n in tokens:
        enc = tok(build_prompt(tok, n), return_tensors="pt", truncation=True, max_length=n + 256).to(device)
        ids = enc["input_ids"]
        yield n, capture_cache(model, ids, enc.get("attention_mask")), find_subsequence(ids[0].tolist(), pattern)


def main(argv=None) -> list[dict]:
    ap = argparse.ArgumentParser(description="TurboQuant score-fidelity report (needle in a haystack).")
    ap.add_argument("--model", help="local checkpoint directory (model + tokenizer); default: synthetic caches")
    ap.add_argument("--tokens", type=int, nargs="+", default=[2048, 4096, 8192])
    ap.add_argument("--bits", type=int, nargs="+", default=[2, 3, 4])
    ap.add_argument("--layers", type=int, default=36, help="synthetic: layers")
    ap.add_argument("--heads", type=int, default=2, help="synthetic: kv heads")
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--device", default="cuda" if torch.cuda.is_available() else "cpu")
    ap.add_argument("--json", help="write the reports here as JSON")
    args = ap.parse_args(argv)

    if args.model:
        cases = _model_cases(args.model, args.tokens, args.device)
    else:
        cases = ((n, *synthetic_needle_cache(args.layers, 1, args.heads, n, args.head_dim, device=args.device))
                 for n in args.tokens)
    out = []
    for n, layers, needle in cases:
        seq = layers[0][0].shape[2]
        print("=" * 70)
        print(f"Context: {seq} tokens | Needle at token {needle}")
        print("=" * 70)
        for rep in validate_cache(layers, args.bits, needle):
            print(format_report(rep))
            out.append({"tokens": seq, "needle": needle, **asdict(rep)})
        print()
    if args.json:
        with open(args.json, "w") as f:
            json.dump(out, f, indent=1)
    return out


if __name__ == "__main__":
    main()
