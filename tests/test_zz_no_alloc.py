"""tq_attention_fwd_kv_noalloc: the allocation-free variant of tq_attention_fwd_kv.

Called through the C ABI (ctypes) on the split-K decode path, its outputs must be
bit-identical to tq_attention_fwd_kv given a caller workspace, on two calls in a
row (the second with a smaller input, so it reuses a scratch array that still
holds the first call's partials), and a shape whose partials exceed the array
must be refused with a message.
"""

import math

import pytest
import torch

from turboquant_pytorch import _native
from turboquant_pytorch.compressors import TurboQuantCompressorMSE, TurboQuantCompressorV2, _tables

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _setup(B, hq, hkv, sk, bits, seed, d=128):
    g = torch.Generator(device=DEV).manual_seed(seed)
    q = torch.randn(B, hq, 1, d, device=DEV, generator=g).to(torch.bfloat16)
    k = torch.randn(B, hkv, sk, d, device=DEV, generator=g).to(torch.bfloat16)
    v = torch.randn(B, hkv, sk, d, device=DEV, generator=g).to(torch.bfloat16)
    kc = TurboQuantCompressorV2(d, bits, seed=42, device=DEV)
    vc = TurboQuantCompressorMSE(d, bits, seed=10042, device=DEV)
    ck, cv = kc.compress(k), vc.compress(v)
    q_rot, q_proj = kc.prepare_queries(q)
    return kc, vc, ck, cv, q_rot, q_proj


def _call(noalloc, kc, vc, ck, cv, q_rot, q_proj, causal=0):
    lib = _native.lib()
    B, hq, sq, d = q_rot.shape
    _, hkv, sk, _ = ck["shape"]
    bits = kc.mse_bits + 1
    tk = _tables(kc, q_rot.device, with_qjl=True)
    tv = _tables(vc, q_rot.device, with_qjl=False)
    out = torch.full((B, sq, hq, d), float("nan"), dtype=torch.float32, device=DEV)
    args = [q_rot.data_ptr(), q_proj.data_ptr(), ck["packed_key_indices"].data_ptr(),
            ck["packed_qjl_signs"].data_ptr(), ck["residual_norm"].data_ptr(), ck["vec_norms"].data_ptr(),
            tk.cent16.data_ptr(), bits, cv["packed_indices"].data_ptr(), cv["vec_norms"].data_ptr(),
            tv.cent32.data_ptr(), vc.bits, tv.pit_split.data_ptr(), B, hq, hkv, sq, sk, sk, d,
            math.sqrt(math.pi / 2) / d, 1 / math.sqrt(d), causal, None, 0, 0, 0, 0, out.data_ptr(),
            _native.TQ_F32, out.stride(0), out.stride(2), out.stride(1)]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        st = lib.tq_attention_fwd_kv_noalloc(*args, stream)
    else:
        nbytes = lib.tq_attention_workspace_size(B, hq, hkv, sq, sk, d, bits)
        assert nbytes > 0  # the split-K decode path, the one that uses scratch
        ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
        st = lib.tq_attention_fwd_kv(*args, ws.data_ptr(), nbytes, stream)
    _native.check(st, "noalloc" if noalloc else "workspace")
    torch.cuda.synchronize()
    return out


def test_noalloc_matches_workspace_entry_point_twice():
    print("case: noalloc two calls (16 x 32768 then 2 x 5000)", flush=True)
    assert _native.lib().tq_noalloc_scratch_bytes() == 16 << 20
    big = _setup(16, 32, 8, 32768, 3, seed=1)
    small = _setup(2, 8, 2, 5000, 4, seed=2)
    a1 = _call(True, *big)
    b1 = _call(False, *big)
    assert torch.isfinite(a1).all() and torch.equal(a1, b1)
    a2 = _call(True, *small)
    b2 = _call(False, *small)
    assert torch.isfinite(a2).all() and torch.equal(a2, b2)
    # and back to the first shape, causal, after the smaller call's partials
    assert torch.equal(_call(True, *big, causal=1), _call(False, *big, causal=1))


def test_noalloc_head_dim64_matches_workspace_entry_point():
    """Head_dim 64 on the decode kernels: few splits (the split merge of any head dim), many
    splits (the per-column merge) and the table kernel (bits 4), each against the workspace
    entry point, in a row on the one scratch array."""
    print("case: noalloc head_dim 64 (16 x 32768 bits 3, 1 x 20000 MHA bits 3, 2 x 5000 bits 4)", flush=True)
    for shape in ((16, 32, 8, 32768, 3, 5), (1, 12, 12, 20000, 3, 6), (2, 8, 2, 5000, 4, 7)):
        case = _setup(*shape, d=64)
        a = _call(True, *case)
        b = _call(False, *case)
        assert torch.isfinite(a).all() and torch.equal(a, b), shape


def test_noalloc_refuses_shapes_beyond_the_scratch_array():
    print("case: noalloc too large", flush=True)
    lib = _native.lib()
    # 2048 (batch, kv head) sequences x 16 query columns: at least 2048 split records of
    # 16 x 130 f32 (17 MB)
    B, hq, hkv, sk, d, bits = 128, 256, 16, 4096, 128, 3
    need = lib.tq_attention_workspace_size(B, hq, hkv, 1, sk, d, bits)
    assert need > lib.tq_noalloc_scratch_bytes()
    z = torch.zeros(16, dtype=torch.uint8, device=DEV)
    p = z.data_ptr()
    st = lib.tq_attention_fwd_kv_noalloc(p, p, p, p, p, p, p, bits, p, p, p, bits, p, B, hq, hkv, 1, sk, sk, d,
                                         0.1, 0.1, 0, None, 0, 0, 0, 0, p, _native.TQ_F32, 0, 0, 0,
                                         torch.cuda.current_stream().cuda_stream)
    assert st == -1 and b"scratch" in lib.tq_last_error()
