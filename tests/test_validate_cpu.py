"""Validation metrics harness (reference: validate.py:115-225, tests/test_slow.py:79-93).

Each metric is pinned against a numpy brute-force computation on the same score
vectors (stable descending sort for ranks), the byte accounting against the
hand-counted bit budget per vector, and the synthetic needle cache against its
own construction (the needle is the exact top-1 key).
"""

import json

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from turboquant_pytorch import validate as V


@pytest.mark.parametrize("bits,key_bits,value_bits", [(2, 128 + 128 + 32, 256 + 16),
                                                      (3, 256 + 128 + 32, 384 + 16),
                                                      (4, 384 + 128 + 32, 512 + 16)])
def test_storage_bits_per_vector(bits, key_bits, value_bits):
    assert V.storage_bits(1, 128, bits) == (key_bits, value_bits)
    assert V.storage_bits(10, 128, bits) == (10 * key_bits, 10 * value_bits)


def test_storage_bits_one_bit_keys_floor():
    # bits=1 keeps 1-bit key codes (max(bits-1, 1))
    assert V.storage_bits(1, 64, 1) == (64 + 64 + 32, 64 + 16)


def _np_metrics(real, est, needle):
    cos, t1, t5, rk = [], [], [], []
    for r, e in zip(real, est):
        cos.append(O.cosine(r.astype(np.float64), e.astype(np.float64)))
        a = int(np.argmax(r))
        t1.append(a == int(np.argmax(e)))
        order = np.argsort(-e.astype(np.float64), kind="stable")
        t5.append(a in order[:5].tolist())
        rk.append(int(np.nonzero(order == needle)[0][0]))
    return np.array(cos), np.array(t1), np.array(t5), np.array(rk)


def test_score_metrics_match_bruteforce():
    g = torch.Generator().manual_seed(0)
    real = torch.randn(3, 4, 1, 300, generator=g)
    est = real + 0.3 * torch.randn(3, 4, 1, 300, generator=g)
    est = torch.round(est * 8) / 8  # plenty of ties, including at the needle
    m = V.score_metrics(real, est, needle=17)
    cos, t1, t5, rk = _np_metrics(real.reshape(12, 300).numpy(), est.reshape(12, 300).numpy(), 17)
    assert np.allclose(m.cosine.numpy(), cos, atol=1e-6)
    assert (m.top1.numpy() == t1).all() and (m.top5.numpy() == t5).all()
    assert (m.needle_rank.numpy() == rk).all()
    assert 0 < t1.sum() < 12  # the case exercises both outcomes


def test_score_metrics_known_answers():
    real = torch.tensor([[0., 5., 1., 2., 3., 4., -1.]])
    est = torch.tensor([[9., 4., 9., 1., 0., 3., 2.]])
    m = V.score_metrics(real, est, needle=2)
    # exact top-1 is key 1; the estimate's top-1 is key 0 (first of the tied maxima)
    assert not bool(m.top1[0])
    # estimate's descending order: 0, 2 (tie broken by position), 1, 5, 6, 3, 4 -> key 1 in top 5
    assert bool(m.top5[0]) and int(m.needle_rank[0]) == 1
    assert V.score_metrics(real, real, needle=1).needle_rank.item() == 0
    assert V.score_metrics(real, real).cosine.item() == pytest.approx(1.0)
    with pytest.raises(ValueError):
        V.score_metrics(real, est, needle=7)
    with pytest.raises(ValueError):
        V.score_metrics(real, est[:, :6])


def test_score_variance_matches_numpy():
    s = torch.randn(2, 3, 4, 50, generator=torch.Generator().manual_seed(1))
    ref = s.numpy().astype(np.float64).var(axis=-1, ddof=1).mean(axis=(0, 2))
    assert np.allclose(V.score_variance(s).numpy(), ref, rtol=1e-5)


def test_find_subsequence_exact_and_prefix():
    ids = [5, 1, 2, 3, 9, 1, 2, 3, 4]
    assert V.find_subsequence(ids, [1, 2, 3, 4]) == 5
    assert V.find_subsequence(ids, [1, 2, 3, 7]) == 1   # longest prefix found
    assert V.find_subsequence(ids, [8, 8]) is None


class _CharTokenizer:
    chat_template = None

    def encode(self, text, add_special_tokens=True):
        return [ord(c) for c in text]


def test_build_prompt_places_needle():
    tok = _CharTokenizer()
    p = V.build_prompt(tok, target_tokens=10 * len(V.HAYSTACK), needle_pos=0.3)
    assert p.count(V.HAYSTACK) == 10 and p.count(V.NEEDLE) == 1
    assert p.index(V.NEEDLE) == 3 * len(V.HAYSTACK) + len("\n--- Memo ---\n")
    assert p.endswith(V.QUESTION)


def test_synthetic_needle_is_exact_top1():
    layers, needle = V.synthetic_needle_cache(n_layers=3, heads=4, seq=4096, dtype=torch.float32)
    assert needle == 2047
    for k, v in layers:
        q = k[:, :, -1:]
        s = (q @ k.transpose(-1, -2))[:, :, 0]
        assert (s.argmax(-1) == needle).all()
        assert v.shape == k.shape


def test_validate_cache_cpu_and_cli(tmp_path):
    layers, needle = V.synthetic_needle_cache(n_layers=2, heads=2, seq=512, head_dim=64)
    reps = V.validate_cache(layers, (2, 3, 4), needle, with_variance=True)
    for rep in reps:
        kb, vb = V.storage_bits(2 * 512, 64, rep.bits)
        assert rep.compressed_bytes == 2 * (kb + vb) / 8
        assert rep.uncompressed_bytes == 2 * 2 * (2 * 512 * 64) * 2
        assert rep.ratio == pytest.approx(rep.uncompressed_bytes / rep.compressed_bytes)
        assert rep.n_checks == 4 and set(rep.variance) == {0, 1}
    cos = [r.cosine for r in reps]
    assert cos[0] < cos[1] < cos[2] and cos[1] > 0.98
    assert reps[2].top5_pct == 100.0 and reps[2].needle_rank < 1.0
    out = tmp_path / "v.json"
    recs = V.main(["--tokens", "256", "--bits", "3", "--layers", "2", "--heads", "2", "--head-dim", "64",
                   "--device", "cpu", "--json", str(out)])
    assert json.loads(out.read_text()) == json.loads(json.dumps(recs))
    assert recs[0]["tokens"] == 256 and recs[0]["bits"] == 3
