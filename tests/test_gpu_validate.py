"""Validation harness on the GPU path (packed planes, fused score kernels).

The on-device metrics must equal a numpy brute force over the same score
vectors; the stored bytes must equal the packed plane sizes (52 + 50 B per
key/value vector at d=128, bits=3).
"""

import numpy as np
import pytest
import torch

from oracle import tq_oracle as O
from turboquant_pytorch import validate as V
from turboquant_pytorch.compressors import TurboQuantCompressorV2

pytestmark = pytest.mark.gpu


def test_gpu_metrics_match_bruteforce():
    print("case: validate metrics gpu", flush=True)
    layers, needle = V.synthetic_needle_cache(n_layers=1, heads=8, seq=2048, device="cuda")
    k = layers[0][0]
    kc = TurboQuantCompressorV2(128, 3, seed=0, device="cuda")
    q = k[:, :, -1:]
    real = torch.matmul(q.float(), k.float().transpose(-2, -1))
    est = kc.asymmetric_attention_scores(q, kc.compress(k))
    m = V.score_metrics(real, est, needle)
    r, e = real.reshape(8, -1).cpu().numpy(), est.reshape(8, -1).cpu().numpy()
    for i in range(8):
        assert abs(m.cosine[i].item() - O.cosine(r[i].astype(np.float64), e[i].astype(np.float64))) < 1e-5
        order = np.argsort(-e[i].astype(np.float64), kind="stable")
        a = int(np.argmax(r[i]))
        assert bool(m.top1[i]) == (a == int(np.argmax(e[i])))
        assert bool(m.top5[i]) == (a in order[:5].tolist())
        assert int(m.needle_rank[i]) == int(np.nonzero(order == needle)[0][0])


def test_gpu_validate_report():
    print("case: validate report gpu", flush=True)
    layers, needle = V.synthetic_needle_cache(n_layers=3, heads=2, seq=4096, device="cuda")
    reps = V.validate_cache(layers, (2, 3, 4), needle)
    per_vec = {2: (16 + 16 + 4) + (32 + 2), 3: (32 + 16 + 4) + (48 + 2), 4: (48 + 16 + 4) + (64 + 2)}
    for rep in reps:
        assert rep.packed_bytes == 3 * 2 * 4096 * per_vec[rep.bits]
        assert rep.n_checks == 6
    assert [round(r.ratio, 2) for r in reps] == [7.31, 5.02, 3.82]
    assert reps[0].cosine < reps[1].cosine < reps[2].cosine and reps[1].cosine > 0.99
    assert reps[2].top1_pct == 100.0 and reps[2].needle_rank == 0.0
