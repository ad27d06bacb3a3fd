"""The compressed KV cache on the GPU: in-place appends and kv_stride attention.

The cache's planes must equal a one-shot compression of the concatenated
sequence bit for bit, and attention read through kv_stride from the capacity
planes must equal attention over compact planes exactly (same kernels, same
data).  End to end, cached greedy decoding must follow the cache-less
recomputation the reference performs.
"""

import math

import pytest
import torch

from oracle import tq_oracle as O
from transformers_turboquant import TurboQuantCache, apply_turboquant
from turboquant_pytorch import _native
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2, _tables
from turboquant_pytorch.fused import compressed_attention

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bits", [2, 3, 4])
def test_cache_planes_and_attention_match_compact(bits):
    print("case: cache planes bits", bits, flush=True)
    dev, d, B, Hkv, G = "cuda", 128, 2, 2, 4
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=dev)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=dev)
    g = torch.Generator(device=dev).manual_seed(0)
    total = 100 + 5 + 300
    k = torch.randn(B, Hkv, total, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, total, d, device=dev, generator=g).to(torch.bfloat16)
    cache = TurboQuantCache()
    steps = [(0, 100)] + [(100 + i, 101 + i) for i in range(5)] + [(105, total)]
    for lo, hi in steps:
        ck, cv = cache.append(0, kc, vc, k[:, :, lo:hi], v[:, :, lo:hi])
        lay = cache.layer(0)
        assert ck["shape"] == (B, Hkv, hi, d) and ck["kv_stride"] == lay.capacity >= hi
        fk, fv = kc.compress(k[:, :, :hi]), vc.compress(v[:, :, :hi])
        n = B * Hkv * hi
        got_k, got_v = lay.compact()
        for name in ("packed_key_indices", "packed_qjl_signs"):
            assert torch.equal(got_k[name], fk[name]), name
        assert torch.equal(got_k["residual_norm"], fk["residual_norm"])
        assert torch.equal(got_k["vec_norms"], fk["vec_norms"])
        assert torch.equal(got_v["packed_indices"], fv["packed_indices"])
        assert torch.equal(got_v["vec_norms"], fv["vec_norms"].reshape(n))
        # one decode row (split-K decode kernels) and 40 causal rows (tiled kernel)
        for sq in (1, 40) if hi >= 40 else (1,):
            q = torch.randn(B, Hkv * G, sq, d, device=dev, generator=g).to(torch.bfloat16)
            a = compressed_attention(q, kc, vc, ck, cv, causal=True, out_dtype=torch.float32)
            c = compressed_attention(q, kc, vc, fk, fv, causal=True, out_dtype=torch.float32)
            torch.cuda.synchronize()
            assert torch.equal(a, c), (hi, sq)
    assert cache.layer(0).capacity == 512  # 256 -> grown by doubling


def test_scores_kv_stride_match_compact():
    print("case: scores kv_stride", flush=True)
    dev, d, B, Hkv, G, bits = "cuda", 128, 2, 2, 4, 3
    kc = TurboQuantCompressorV2(d, bits, seed=7, device=dev)
    vc = TurboQuantCompressorMSE(d, bits, seed=10007, device=dev)
    g = torch.Generator(device=dev).manual_seed(1)
    k = torch.randn(B, Hkv, 333, d, device=dev, generator=g)
    cache = TurboQuantCache()
    ck, _ = cache.append(0, kc, vc, k, k)
    fk = kc.compress(k)
    lib = _native.lib()
    t = _tables(kc, dev, with_qjl=True)
    coeff = math.sqrt(math.pi / 2) / d
    for sq in (1, 3, 33):
        q = torch.randn(B, Hkv * G, sq, d, device=dev, generator=g)
        q_rot, q_proj = kc.prepare_queries(q)
        outs = []
        for planes, stride in ((ck, ck["kv_stride"]), (fk, 0)):
            o = torch.empty(B, Hkv * G, sq, 333, device=dev)
            _native.check(lib.tq_attention_scores_kv(
                q_rot.data_ptr(), q_proj.data_ptr(), planes["packed_key_indices"].data_ptr(),
                planes["packed_qjl_signs"].data_ptr(), planes["residual_norm"].data_ptr(),
                planes["vec_norms"].data_ptr(), t.cent16.data_ptr(), B, Hkv * G, Hkv, sq, 333, stride, d,
                bits, coeff, o.data_ptr(), _native.stream_of(o)), "scores_kv")
            outs.append(o)
        torch.cuda.synchronize()
        assert torch.equal(outs[0], outs[1]), sq
        # the compressor's method reads kv_stride from the cache dict
        assert torch.equal(kc.asymmetric_attention_scores(q, ck), kc.asymmetric_attention_scores(q, fk))
        # and the oracle's estimator on the same packed planes and prepared queries
        n = B * Hkv * 333
        codes = O.unpack_bits(fk["packed_key_indices"].reshape(n, -1).cpu().numpy(), bits - 1, d)
        signs = O.unpack_bits(fk["packed_qjl_signs"].reshape(n, -1).cpu().numpy(), 1, d)
        rn = fk["residual_norm"].reshape(n).cpu().numpy()
        vn = fk["vec_norms"].reshape(n).cpu().numpy()
        qr, qp = q_rot.cpu().numpy(), q_proj.cpu().numpy()
        cent = t.cent16.cpu().numpy()
        for b in range(B):
            for h in range(Hkv * G):
                r = slice((b * Hkv + h // G) * 333, (b * Hkv + h // G + 1) * 333)
                ref = O.scores_packed(qr[b, h], qp[b, h], codes[r], signs[r], rn[r], vn[r], cent, coeff)
                assert O.rel_err(outs[0][b, h].cpu().numpy(), ref) < 1e-5, (sq, b, h)
    # a stride below Sk is rejected
    bad = lib.tq_attention_scores_kv(q_rot.data_ptr(), q_proj.data_ptr(), fk["packed_key_indices"].data_ptr(),
                                     fk["packed_qjl_signs"].data_ptr(), fk["residual_norm"].data_ptr(),
                                     fk["vec_norms"].data_ptr(), t.cent16.data_ptr(), B, Hkv * G, Hkv, 33, 333,
                                     100, d, bits, coeff, outs[0].data_ptr(), None)
    assert bad != 0 and b"kv_stride" in lib.tq_last_error()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cached_generate_matches_recompute_gpu(dtype):
    print("case: cached generate", dtype, flush=True)
    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(0)
    cfg = LlamaConfig(vocab_size=1000, hidden_size=1024, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2)  # head_dim 128, G = 4: decode kernels
    # causal="auto": token-by-token decoding is causal, so the recomputation must be too
    model = apply_turboquant(LlamaForCausalLM(cfg).eval(), bits=3, causal="auto").to("cuda", dtype)
    ids = torch.randint(0, 1000, (2, 37), generator=torch.Generator().manual_seed(5)).cuda()
    kw = dict(max_new_tokens=8, min_new_tokens=8, do_sample=False, output_logits=True,
              return_dict_in_generate=True, attention_mask=torch.ones_like(ids))
    with torch.no_grad():
        ref = model.generate(ids, use_cache=False, **kw)
        cache = TurboQuantCache()
        got = model.generate(ids, use_cache=True, past_key_values=cache, **kw)
    assert cache.get_seq_length() == 37 + 7
    # the cached path runs the split-K decode kernels, the recomputation the tiled
    # kernel: the same estimator with different f16 roundings of P.  Raw logits,
    # since min_new_tokens writes -inf into the processed scores.
    assert len(got.logits) == len(ref.logits) == 8
    cos = [O.cosine(a.float().cpu().numpy(), b.float().cpu().numpy()) for a, b in zip(got.logits, ref.logits)]
    assert min(cos) > (0.9999 if dtype == torch.float32 else 0.999), cos
    assert (got.sequences == ref.sequences).float().mean() > 0.95


@pytest.mark.parametrize("d,bits,dt,B,H,Hq,S,cap,pos", [
    (128, 3, torch.bfloat16, 1, 8, 32, 1, 4096, 4095),   # one decode step (one launch: K, V and Q)
    (128, 2, torch.float32, 2, 3, 6, 37, 300, 17),
    (128, 4, torch.float16, 2, 2, 8, 5, 256, 100),
    (64, 3, torch.bfloat16, 2, 12, 12, 19, 64, 45),
    (128, 3, torch.bfloat16, 2, 8, 32, 3000, 3500, 311),  # more blocks than the device holds: shared
    (96, 3, torch.bfloat16, 2, 2, 4, 9, 40, 3),           # tile kernels: other head dims
    (80, 2, torch.float32, 1, 3, 3, 7, 20, 13),
])
def test_cache_append_writes_the_compressors_rows(d, bits, dt, B, H, Hq, S, cap, pos):
    """tq::cache_append (tq_cache_append) writes rows [pos, pos + S) of each (batch, kv head) of
    the capacity planes exactly as compress() packs those rows, leaves every other row alone, and
    prepares the queries exactly as prepare_queries() does."""
    print(f"case: cache_append d={d} bits={bits} dt={dt} B={B} H={H} Hq={Hq} S={S} cap={cap} pos={pos}", flush=True)
    from turboquant_pytorch._ops import ops

    dev = "cuda"
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=dev)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=dev)
    g = torch.Generator(device=dev).manual_seed(S + d)
    k = torch.randn(B, S, H, d, device=dev, generator=g).to(dt).transpose(1, 2)  # strided, as the families pass
    v = torch.randn(B, H, S, d, device=dev, generator=g).to(dt)
    q = torch.randn(B, Hq, S, d, device=dev, generator=g).to(dt)
    fk, fv = kc.compress(k), vc.compress(v)
    q_rot_ref, q_proj_ref = kc.prepare_queries(q)
    kw, vw = fk["packed_key_indices"].shape[-1], fv["packed_indices"].shape[-1]
    fill = 0xA5
    planes = {
        "kcodes": torch.full((B, H, cap, kw), fill, dtype=torch.uint8, device=dev),
        "ksigns": torch.full((B, H, cap, d // 8), fill, dtype=torch.uint8, device=dev),
        "krn": torch.full((B, H, cap), 7.0, dtype=torch.float16, device=dev),
        "kvn": torch.full((B, H, cap), 7.0, dtype=torch.float16, device=dev),
        "vcodes": torch.full((B, H, cap, vw), fill, dtype=torch.uint8, device=dev),
        "vvn": torch.full((B, H, cap), 7.0, dtype=torch.float16, device=dev),
    }
    before = {n: t.clone() for n, t in planes.items()}
    tk, tv = _tables(kc, dev, with_qjl=True), _tables(vc, dev, with_qjl=False)
    q_rot, q_proj = ops().cache_append(k, v, q, tk.pi_split, tk.seff_split, tk.cent32, tk.bounds32, kc.mse_bits,
                                       tv.pi_split, tv.bounds32, vc.bits, tk.s_eff16, planes["kcodes"],
                                       planes["ksigns"], planes["krn"], planes["kvn"], planes["vcodes"],
                                       planes["vvn"], pos)
    torch.cuda.synchronize()
    sl = slice(pos, pos + S)
    want = {
        "kcodes": fk["packed_key_indices"].reshape(B, H, S, kw), "ksigns": fk["packed_qjl_signs"].reshape(B, H, S, -1),
        "krn": fk["residual_norm"].reshape(B, H, S), "kvn": fk["vec_norms"].reshape(B, H, S),
        "vcodes": fv["packed_indices"].reshape(B, H, S, vw), "vvn": fv["vec_norms"].reshape(B, H, S),
    }
    for name, t in planes.items():
        assert torch.equal(t[:, :, sl], want[name]), name
        rest = torch.ones(cap, dtype=torch.bool, device=dev)
        rest[sl] = False
        assert torch.equal(t[:, :, rest], before[name][:, :, rest]), name
    assert torch.equal(q_rot, q_rot_ref) and torch.equal(q_proj, q_proj_ref)
    # without queries: the same rows, and empty query outputs
    for name, t in planes.items():
        t.copy_(before[name])
    e_rot, e_proj = ops().cache_append(k, v, None, tk.pi_split, tk.seff_split, tk.cent32, tk.bounds32, kc.mse_bits,
                                       tv.pi_split, tv.bounds32, vc.bits, tk.s_eff16, planes["kcodes"],
                                       planes["ksigns"], planes["krn"], planes["kvn"], planes["vcodes"],
                                       planes["vvn"], pos)
    torch.cuda.synchronize()
    assert e_rot.numel() == 0 and e_proj.numel() == 0
    for name, t in planes.items():
        assert torch.equal(t[:, :, sl], want[name]), name


def test_cached_decode_step_uses_one_append_launch():
    """A patched layer's decode step with a TurboQuantCache: the appended planes equal a one-shot
    compression and the output equals compressed_attention on the compact planes."""
    print("case: decode step through the cache", flush=True)
    dev, d, B, Hkv, G, bits = "cuda", 128, 1, 8, 4, 3
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=dev)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=dev)
    g = torch.Generator(device=dev).manual_seed(3)
    total = 600
    k = torch.randn(B, Hkv, total, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, total, d, device=dev, generator=g).to(torch.bfloat16)
    cache = TurboQuantCache()
    cache.append(0, kc, vc, k[:, :, :599], v[:, :, :599])
    q = torch.randn(B, Hkv * G, 1, d, device=dev, generator=g).to(torch.bfloat16)
    ck, cv, q_rot, q_proj = cache.append_prepare(0, kc, vc, k[:, :, 599:], v[:, :, 599:], q)
    from turboquant_pytorch.fused import attention_from_prepared
    got = attention_from_prepared(q_rot, q_proj, kc, vc, ck, cv, out_dtype=torch.float32)
    fk, fv = kc.compress(k), vc.compress(v)
    ref = compressed_attention(q, kc, vc, fk, fv, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("d,bits,Hkv,G", [(128, 3, 8, 4), (64, 3, 12, 1), (64, 4, 2, 8), (128, 2, 2, 8)])
def test_append_attend_matches_append_prepare_then_attention(d, bits, Hkv, G):
    """TurboQuantCache.append_attend (one tq::cache_attend call) against append_prepare followed
    by attention_from_prepared on a copy of the same cache: the same output and cache planes, bit
    for bit, over several decode steps (causal, with a padding mask on the last one)."""
    print("case: append_attend", dict(d=d, bits=bits, Hkv=Hkv, G=G), flush=True)
    from turboquant_pytorch.fused import attention_from_prepared

    dev, B = "cuda", 2
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=dev)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=dev)
    g = torch.Generator(device=dev).manual_seed(d + bits)
    total = 1500
    k = torch.randn(B, Hkv, total, d, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, total, d, device=dev, generator=g).to(torch.bfloat16)
    a, b = TurboQuantCache(), TurboQuantCache()
    for c in (a, b):
        c.append(0, kc, vc, k[:, :, :1496], v[:, :, :1496])
    for pos in range(1496, total):
        q = torch.randn(B, Hkv * G, 1, d, device=dev, generator=g).to(torch.bfloat16)
        mask = None
        if pos == total - 1:
            mask = torch.zeros(B, 1, 1, pos + 1, device=dev)
            mask[0, 0, 0, :100] = torch.finfo(torch.float32).min
        got = a.append_attend(0, kc, vc, k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], q, attention_mask=mask,
                              causal=True, out_dtype=torch.bfloat16)
        ck, cv, q_rot, q_proj = b.append_prepare(0, kc, vc, k[:, :, pos:pos + 1], v[:, :, pos:pos + 1], q)
        want = attention_from_prepared(q_rot, q_proj, kc, vc, ck, cv, attention_mask=mask, causal=True,
                                       out_dtype=torch.bfloat16)
        torch.cuda.synchronize()
        assert torch.isfinite(got.float()).all() and torch.equal(got, want), pos
    la, lb = a.layer(0), b.layer(0)
    assert la.length == lb.length == total
    for name in la.kp:
        assert torch.equal(la.kp[name], lb.kp[name]), name
    for name in la.vp:
        assert torch.equal(la.vp[name], lb.vp[name]), name
