"""A decode step captured into a HIP graph (torch.cuda.CUDAGraph on ROCm) replays exactly.

The step is what a serving loop launches per layer and token: compress the new token's
K and V, prepare the query, and run split-K decode attention over a compressed cache.
Its entry points allocate nothing inside the library and record no memset or host
synchronisation, so the whole step can be captured once and replayed, which removes
the per-launch host cost that dominates short-context decoding.  Every replay, with new
inputs copied in and eager work and synchronisations in between, must equal the eager
step bit for bit (same kernels, same data, no atomics).
"""

import pytest
import torch

from turboquant_pytorch import compressed_attention
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("sk,d,bits", [(700, 128, 3), (5000, 128, 3), (5000, 64, 3), (20000, 64, 4)])
def test_decode_step_graph_replays_match_eager(sk, d, bits):
    print("case: graph decode step sk", sk, "d", d, "bits", bits, flush=True)
    B, Hkv, G = 2, 8, 4
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(9)
    ck = kc.compress(torch.randn(B, Hkv, sk, d, device=DEV, generator=g).to(torch.bfloat16))
    cv = vc.compress(torch.randn(B, Hkv, sk, d, device=DEV, generator=g).to(torch.bfloat16))
    k_new = torch.empty(B, Hkv, 1, d, device=DEV, dtype=torch.bfloat16)
    v_new = torch.empty_like(k_new)
    q = torch.empty(B, Hkv * G, 1, d, device=DEV, dtype=torch.bfloat16)

    def fill():
        k_new.copy_(torch.randn(k_new.shape, device=DEV, generator=g))
        v_new.copy_(torch.randn(v_new.shape, device=DEV, generator=g))
        q.copy_(torch.randn(q.shape, device=DEV, generator=g))

    def step():
        nk, nv = kc.compress(k_new), vc.compress(v_new)
        o = compressed_attention(q, kc, vc, ck, cv, causal=True, out_dtype=torch.float32)
        return nk["packed_key_indices"], nk["packed_qjl_signs"], nk["residual_norm"], nv["packed_indices"], o

    fill()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside capture: tables, occupancy queries
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for rep in range(4):
        fill()
        torch.cuda.synchronize()
        want = [t.clone() for t in step()]
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for got, ref in zip(captured, want):
            assert torch.equal(got, ref), rep
